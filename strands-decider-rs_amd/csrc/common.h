// Shared definitions of the gfx950 engine: vector types, error checks, and the launcher
// functions each kernel file exports to the engine (engine.cpp drives every kernel through these).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace sd {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

#define SD_HIP(call)                                                                                   \
    do {                                                                                               \
        hipError_t e_ = (call);                                                                        \
        if (e_ != hipSuccess)                                                                          \
            throw ::sd::Error(std::string(#call) + ": " + hipGetErrorString(e_) + " (" + __FILE__ + ":" + \
                              std::to_string(__LINE__) + ")");                                         \
    } while (0)

#define SD_CHECK(cond, msg)                          \
    do {                                             \
        if (!(cond)) throw ::sd::Error(std::string(msg)); \
    } while (0)

// Launch-time bookkeeping shared with the engine: every kernel launch goes through `launched`
// so a failed launch is reported at its call site.
void launched(const char* what);

// Kernel-own timing for Engine::profile: while a step runs with this slot set, the first GEMM it
// launches goes through hipExtLaunchKernel, which records the kernel's own start and end in
// `start` / `stop` (the event pair around a step would add the dispatch of the launch).
struct KernelEvents {
    hipEvent_t start = nullptr, stop = nullptr;
    int launches = 0;
};
KernelEvents*& kernel_events();

// 8-bit scale codes -> f16 bits (src/model.rs:217-236); host only (engine.cpp).
void decode_scale_codes(const uint8_t* src, size_t n, size_t g, uint16_t* dst, std::vector<double>& pw);

// ---- quantized matmul (gemm.hip) -----------------------------------------------------------
// Y[M,N] f16 = A[M,K] f16 . deq(W[N,K])^T with W int4 group-32 symmetric in the reference's
// block layout ([N][K/32] blocks of 4 u32, k = 8w + e of a block in word w, value (q-8)*scale,
// scales [N][K/32] f16) with the nibbles of each word in the engine order of repack_w4.  `exact` selects the f32-dequant arithmetic of the reference's GEMV
// path (used for M <= 20), otherwise the f16 dequant of its tiled path.  With `part` non-null the
// k range is split over ks workgroups that write f32 partials part[ks][M][N] instead of Y (ks = 1
// allowed); the consumer sums them in slot order (add_norm, or reduce_partials).  cfg < 0 picks
// the tile shape by M.
// `tiled`: W and S are in the tiled layout of tile_w4.
void gemm_w4(const f16* A, const uint32_t* W, const f16* S, f16* Y, float* part, int M, int N, int K, bool exact,
             int ks, hipStream_t st, int cfg = -1, bool tiled = false);
// Whether tile_w4 takes an N x K matrix (N a multiple of 32, K of 64).
bool w4_tileable(int N, int K);
// Rewrites a matrix's words (already in the engine nibble order) and scales in place into the tiled
// layout: each tile of 32 columns x 64 k (2 blocks per column) becomes one contiguous KiB of words,
// block (n, b) at 16-byte index ((n / 32) * (K / 64) + b / 2) * 64 + (n % 32) * 2 + b % 2, its
// scale at the same f16 index.  tmp holds N*K/2 + N*K/16 bytes.
void tile_w4(uint32_t* W, f16* S, int N, int K, void* tmp, hipStream_t st);
int gemm_w4_configs();
int gemm_w4_cfg(int M, bool exact);
// Kernel configuration and split-K count for an M x N x K product.  partial_ok: the consumer can
// sum f32 split-K slots (else ks = 1 and the output is f16).
struct GemmPlan {
    int cfg, ks;
};
GemmPlan gemm_w4_plan(int M, int N, int K, bool exact, bool partial_ok, size_t max_part_elems);
// Split count that brings the grid to about target_groups workgroups (power of 2, <= 8).
int gemm_w4_split(int M, int N, int K, int cfg, int target_groups, size_t max_part_elems);
void reduce_partials(const float* part, int ks, size_t n, f16* Y, hipStream_t st);
// Rewrites `words` int4 weight words in place from the reference's nibble order (the model file's)
// to the one every gemm_w4 kernel reads; run once per weight matrix.
void repack_w4(uint32_t* W, size_t words, hipStream_t st);
// gate_up [2I][K] (weights and scales) rewritten in place with its rows interleaved in groups of
// 16: rows 32p .. 32p + 15 = gate rows 16p .., rows 32p + 16 .. = the matching up rows.  tmp holds
// N*K/2 + N*K/16 bytes.
void interleave_gate_up(uint32_t* W, f16* S, int N, int K, void* tmp, hipStream_t st);
// mid[M][N/2] f16 = silu(g) * u of the unsplit gate_up product A . deq(W)^T, W interleaved as above
// (f16 dequant, a 32x32-tile configuration of gemm_w4_plan); N a multiple of 32, K of 256.
void gemm_w4_silu(const f16* A, const uint32_t* W, const f16* S, f16* mid, int M, int N, int K, hipStream_t st,
                  int cfg, bool tiled);
// Whether configuration cfg has the SiLU * mul epilogue of gemm_w4_silu.
bool gemm_w4_has_silu(int cfg);

// ---- quantized GEMV (gemv.hip) ---------------------------------------------------------------
// Y = A[M,K] f16 . deq(W[N,K])^T with the reference GEMV's f32 dequant (src/kernels.rs:590-635) for
// any of its formats (int2/3/4, group a multiple of 32, symmetric or asymmetric with biases Bi).
// `tiled`: W and S in the engine's int4 g32 tiled layout (tile_w4, engine nibble order); else the
// reference's plain layout and bit order.  out: 0 = f16 Y [M][N]; 1 = f32 partial slots Y [ks][M][N]
// (summed in slot order by the consumer); 2 = f16 mid [M][N/2] = silu(gate) * up of a tiled gate_up
// whose rows are interleaved in groups of 16 (interleave_gate_up).
struct GemvPlan {
    int nct = 1, mt = 1, ks = 1;  // column tiles of 16 per workgroup, row tiles of 16, k splits
};
GemvPlan gemv_plan(int M, int N, int K, bool tiled, int out, size_t max_part_elems);
void gemv(const f16* A, const uint32_t* W, const f16* S, const f16* Bi, void* Y, int out, int M, int N, int K, int bits,
          int group, bool asym, bool tiled, const GemvPlan& p, hipStream_t st);

// ---- elementwise / norms (elem.hip) ----------------------------------------------------------
void embed(const uint32_t* ids, int L, const uint32_t* Q, const f16* S, const f16* Bi, int d, int bits,
           int group, bool asym, float* x, hipStream_t st);
// The sublayer output to add: f16 rows y16, or ks f32 partial slots yp[ks][L][d] whose slot-order
// sum rounded to f16 is the same value (null both: no add).
struct YIn {
    const f16* y16 = nullptr;
    const float* yp = nullptr;
    int ks = 0;
    size_t slot = 0;  // elements per slot (L * d)
};
// x[rows[r]] += y, h[r] = rmsnorm(x[rows[r]]) * w -> f16 (h16) or f32 (h32); rows null = identity.
void add_norm(float* x, const YIn& y, const float* w, int d, const uint32_t* rows, int nrows, f16* h16, float* h32,
              hipStream_t st);
// gate_up output in big (f16, [L][2I]) or as ks f32 split-K slots in part; `il`: gate and up
// columns interleaved in groups of 16 (the layout interleave_gate_up gives the weights).
void silu_mul(const f16* big, const float* part, int ks, int L, int I, bool il, f16* mid, hipStream_t st);
// d0[r] = s0[rows[r]] and d1[r] = s1[rows[r]] for r < n, rows of bytes0 / bytes1 (multiples of 16)
void gather_rows2(const void* s0, void* d0, size_t bytes0, const void* s1, void* d1, size_t bytes1, const uint32_t* rows,
                  int n, hipStream_t st);
void add_bias(f16* y, int L, int N, const float* c, hipStream_t st);
void fill_u32(uint32_t* p, size_t n, uint32_t v, hipStream_t st);
// p[0..8) = v[0..8) by a kernel (a value carried in the launch, so the call may be captured)
void set_u32x8(uint32_t* p, const uint32_t v[8], hipStream_t st);
// Several strided device copies in one launch: rows x row_bytes from src (rows src_pitch apart) to
// dst (rows dst_pitch apart).  Pointers, pitches and row_bytes must be multiples of 16 bytes.
struct CopyDesc {
    const uint8_t* src;
    uint8_t* dst;
    uint64_t rows, row_bytes, src_pitch, dst_pitch;
};
void copy_batch(const CopyDesc* d, size_t n, hipStream_t st);

// ---- gated delta net (gdn.hip) ---------------------------------------------------------------
// Several independent token sequences in one forward (the questions of an ask_all, each continuing
// from the same prefix).  Rows of a sequence are consecutive.  Device tables; all null = one
// sequence covering every row:
//   row[r]   = local index i | first row of r's sequence << 16
//   chunk[c] = first row | length << 16 of chunk c (chunks of <= 64 rows never cross sequences)
//   seq[q]   = first chunk | chunk count << 16 of sequence q
//   seq[SD_MAX_SEQS + q] = first row | row count << 16 of sequence q
// The chunk and sequence counts are lu[4] and lu[5].
constexpr int SD_MAX_SEQS = 32;  // sequences per forward
struct Segs {
    const uint32_t* row = nullptr;
    const uint32_t* chunk = nullptr;
    const uint32_t* seq = nullptr;
};

struct GdnShape {
    int H, DK, DV, stride, a_off, b_off, z_off, C;
};

// What a GDN prep needs to compute the causal conv + SiLU of the in_proj rows itself (w null: the
// caller passes the conv output instead).
struct ConvIn {
    const float* w = nullptr;        // [C][4] taps
    const f16* hist = nullptr;       // the live history [3][C]; a prefix snapshot's (named by lu) wins
    const uint32_t* rowt = nullptr;  // per row: index in its sequence | start row << 16 (null: one sequence)
    size_t hist_off = 0;             // the layer's history in a snapshot arena image
};
// Workspace of the chunked recurrence, sized for `cap` tokens: per (chunk, head) the scan's A
// operands split into f16 hi/lo in MFMA fragment order, U (fp32) and e^(G_last).
struct GdnWs {
    f16* wf = nullptr;   // W = T diag(beta e^G) Kn
    f16* qgf = nullptr;  // qn e^G
    f16* qkf = nullptr;  // (qn . kn) e^(G_i - G_j), i >= j
    f16* kgf = nullptr;  // (kn e^(G_last - G))^T
    float* u = nullptr;  // T diag(beta) V, [64][dv] fp32
    float* gl = nullptr; // e^(G_last)
};
size_t gdn_ws_bytes(int cap, const GdnShape& s);
void gdn_ws_carve(void* base, int cap, const GdnShape& s, GdnWs& ws);
// The lu block every plan reads (device, at the start of the pool): u32 [L, P, ctx, has_cache,
// chunks, sequences, 0, 0], then at byte 32 the device address of the prefix snapshot's arena image
// (null: the live arena's states and histories are the prefix).  A layer's state and history sit at
// byte offsets state_off / hist_off of either arena image.
constexpr size_t LU_PREFIX_BYTE = 32;
// Every sequence's first rows read the conv history: the prefix's (lu) or `hist`.
void conv_silu(const f16* big, int stride, int L, int C, const float* w, const f16* hist, float* out,
               const Segs& sg, hipStream_t st, const uint32_t* lu = nullptr, size_t hist_off = 0);
// With cv.w set, q, k and v are the conv + SiLU of big's rows (qkvc unused), else read from qkvc.
// nch = chunk grid size (chunks past lu[4] exit when sg.chunk is set).
void gdn_prep(const float* qkvc, const f16* big, const GdnShape& s, const float* negA, const float* dtb, int L,
              const GdnWs& ws, const ConvIn& cv, const Segs& sg, int nch, const uint32_t* lu, hipStream_t st);
// lu = device block above (the state is loaded when has_cache, from the prefix's arena image when it
// names one); with lu null, load_default decides.  Every sequence starts from that state; the final
// state is written to `state` only for a single sequence (sg.seq null).  nseq = sequence grid size.
// hist (nullable) is updated from big at the end (the reference's hist_update; single sequence
// only), its old rows from the prefix's history.
void gdn_scan(const GdnShape& s, int L, const GdnWs& ws, float* state, const uint32_t* lu, int load_default, float* o,
              const Segs& sg, int nseq, hipStream_t st, size_t state_off = 0, f16* hist = nullptr,
              const f16* big = nullptr, size_t hist_off = 0);
// The same recurrence token by token (the reference's own order), for short inputs: every
// sequence starts from the prefix state as gdn_scan; with one sequence the final state is written
// to `state` and hist (nullable) updated afterwards, as gdn_prep + gdn_scan do.
// With cv.w set, q, k and v are the conv + SiLU of big's rows (qkvc unused; the history is read, so
// hist must be null).
void gdn_recur(const float* qkvc, const f16* big, const GdnShape& s, const float* negA, const float* dtb, int L,
               float* state, const uint32_t* lu, int load_default, float* o, f16* hist, const Segs& sg, int nseq,
               hipStream_t st, size_t state_off = 0, size_t hist_off = 0, const ConvIn& cv = ConvIn{});
void gnorm(const float* o, const f16* big, const GdnShape& s, const float* w, int L, f16* out, hipStream_t st);

// ---- pointer head (head_gpu.hip) -------------------------------------------------------------
// Device copies of head.safetensors (all f32): LayerNorm weight/bias [d], q and k [dim][d] + bias.
struct HeadW {
    const float *nw = nullptr, *nb = nullptr, *qw = nullptr, *qb = nullptr, *kw = nullptr, *kb = nullptr;
    int dim = 0;
};
// proj[r][0..dim) = (answer row ? q : k) projection of LayerNorm(hidden[r]), f64.
void head_rows(const float* hidden, int n_rows, int d, const HeadW& w, const uint8_t* is_answer, double* proj,
               hipStream_t st);
// Question q: option rows [first, first + n) and answer row first + n (qtab[q] = first | n << 16);
// probs[ooff[q] + i] = softmax_i(k_i . q * scale[q]).
void head_probs(const double* proj, int dim, const uint32_t* qtab, const double* scale, const uint32_t* ooff, int nq,
                double* probs, hipStream_t st);
// rows[r] <- unrotate * FWHT(rows[r]) (a rotated torso's output in the head's basis).
void unrotate_rows(float* rows, int n_rows, int d, const double* unrot, hipStream_t st);

// ---- attention (attn.hip) --------------------------------------------------------------------
struct AttnShape {
    int HQ, HK, HD, RD, stride, ctx;
};
// RoPE position of row r = P + its index in its sequence; cache row = P + r.  Q null: the kv heads
// only (attention_split then computes the queries itself).
void qk_prep(const f16* big, const AttnShape& s, const float* qw, const float* kw, const float* rope, int L,
             const uint32_t* lu, const Segs& sg, f16* Q, f16* Kc, f16* Vc, hipStream_t st);
// Workspace (floats) of the key-split path for up to `rows` query rows and 8 splits.
size_t attn_ws_floats(int rows, const AttnShape& s);
// ks = number of key splits (1: no workspace needed; ks > 1 needs rows = L in the workspace).
// Row r attends the prefix (cache rows < P) and its own sequence up to itself.
// Q null: each workgroup computes its queries' RMSNorm (qw) and RoPE (rope, rotary_dim 64) from big.
void attention_split(const f16* Q, const f16* Kc, const f16* Vc, const f16* big, const AttnShape& s, int L,
                     const uint32_t* lu, const Segs& sg, int ks, float* ws, f16* out, hipStream_t st,
                     const float* qw = nullptr, const float* rope = nullptr);

}  // namespace sd
