/*
 * sdhip.h - C ABI of the MI355X (gfx950) engine for the strands-decider torso.
 *
 * This is the drop-in boundary for the reference crate's engine (mircodz/strands-decider-rs,
 * src/engine.rs).  Each entry point below replaces one item of the reference's `Engine` API; the
 * reference item is cited next to it.  A Rust `engine.rs` shim binds these 1:1 (extern "C"
 * declarations of the functions below and a safe wrapper per reference item); the crate's
 * `Decider::new/load/ask/ask_all` (src/lib.rs:113-145) then run unchanged on top.
 *
 * Conventions (as in the reference):
 *  - Functions returning int return 0 on success and nonzero on failure, writing a
 *    NUL-terminated message into err[0..errlen) (the reference's `crate::Error(String)`).
 *  - `sd_engine_forward` is synchronous and exclusive per engine (the reference's `&mut self`):
 *    it returns after the device is idle.  One engine handle must not be used from two threads
 *    at once.
 *  - The engine owns weights, caches and activation buffers; a snapshot owns copies of the
 *    prefix state until `sd_snapshot_free`, and must be freed before its engine; output memory
 *    is caller-owned.
 */
#ifndef SDHIP_H
#define SDHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Context capacity of the KV cache and RoPE table, in tokens (src/engine.rs:16 `CONTEXT`). */
#define SD_CONTEXT 4096

typedef struct sd_engine sd_engine;     /* src/engine.rs:104-132 `Engine` */
typedef struct sd_snapshot sd_snapshot; /* src/engine.rs:81-87 `Snapshot` */
typedef struct sd_head sd_head;         /* src/head.rs:11-14 `Head` */

/* Layer kinds of `Config::layer_types` (src/engine.rs:243-247). */
enum { SD_LINEAR_ATTENTION = 0, SD_FULL_ATTENTION = 1, SD_ADAPTER = 2 };

/* The torso fields of `model::Config` (src/model.rs:31-47). */
typedef struct {
    size_t hidden_size, intermediate_size, n_layers;
    const uint8_t* layer_types; /* n_layers entries: SD_LINEAR_ATTENTION / SD_FULL_ATTENTION / SD_ADAPTER */
    size_t num_attention_heads, num_key_value_heads, head_dim, rotary_dim;
    size_t linear_num_key_heads, linear_key_head_dim, linear_value_head_dim;
    double rope_theta;
    const double* unrotate; /* nullable; hidden_size entries (`Config::unrotate`) */
} sd_config;

/* One manifest tensor, `model::Tensor` (src/model.rs:58-83). */
typedef struct {
    const char* name;
    uint64_t offset, bytes;
    uint32_t N, K, bits, group, asym;
    int32_t had; /* online Hadamard size, -1 when absent (rejected, as in src/engine.rs:248-250) */
} sd_tensor;

/* The embedding rows file, `model::Embed` (src/model.rs:92-103).  Rows are in token-id order, the
 * parts of a row back to back.  With u8 = 1 a row stores its "embed.s" part as 8-bit scale codes (a
 * 4-byte header and one code per scale, decoded at load as `embed_parts` does, src/model.rs:260-283)
 * and is wire_row_bytes long; otherwise rows are row_bytes long (wire_row_bytes 0). */
typedef struct {
    const char* rows_path;
    uint64_t vocab, row_bytes;
    size_t n_parts;
    const char* const* part_names; /* e.g. "embed.q", "embed.s" */
    const uint64_t* part_bytes;    /* bytes per row of each part in GPU layout */
    uint64_t wire_row_bytes;       /* bytes per stored row when they differ from row_bytes, else 0 */
    int32_t u8;                    /* "embed.s" stored as 8-bit scale codes */
} sd_embed;

/* `Engine::load(dir, &Manifest)` (src/engine.rs:175-303): uploads the shards (shard i holds the
 * manifest bytes [shard_starts[i], shard_starts[i] + shard_bytes[i])), the embedding parts, and
 * allocates the recurrent state, conv history and K/V cache. */
int sd_engine_load(const sd_config* cfg, const sd_tensor* tensors, size_t n_tensors, const char* const* shard_paths,
                   const uint64_t* shard_starts, const uint64_t* shard_bytes, size_t n_shards, const sd_embed* embed,
                   sd_engine** out, char* err, size_t errlen);

/* `decode_scales` (src/model.rs:217-236), the load-time decode of 8-bit scale codes: n rows of g
 * codes at src (first a 4-byte header per row: m as f16 bits and j as u16, little-endian; then the
 * n*g codes, sign << 7 | k) into n*g f16 scales (bits) at dst: |scale| = f16(f32(m 2^(-k j / 4096))).
 * src holds src_bytes bytes (at least n * (4 + g)), dst dst_count scales (at least n * g); the power
 * table lives for this call only.  Host only; no device is used. */
int sd_decode_scale_codes(const uint8_t* src, size_t src_bytes, size_t n, size_t g, uint16_t* dst, size_t dst_count,
                          char* err, size_t errlen);

/* Drop of `Engine`. */
void sd_engine_free(sd_engine* e);

/* `Engine::hidden_size` (src/engine.rs:305-307). */
size_t sd_engine_hidden_size(const sd_engine* e);

/* `Engine::adapter` (src/engine.rs:107-108): the device in use, for display. */
const char* sd_engine_adapter(const sd_engine* e);

/* `Engine::forward(ids, rows, cache, keep, timed)` (src/engine.rs:529-662).
 * Runs the torso on ids[0..n), continuing from `cache` (nullable prefix snapshot).  Writes the
 * final hidden rows `rows` (indices into ids) to hidden_out[n_rows * hidden_size] (f32, in the
 * head's basis after the optional unrotate).  gpu_ms (nullable) receives the device time when
 * `timed`, NaN otherwise.  With `keep`, *snap_out receives a snapshot of the prefix + ids. */
int sd_engine_forward(sd_engine* e, const uint32_t* ids, size_t n, const size_t* rows, size_t n_rows,
                      const sd_snapshot* cache, int keep, int timed, float* hidden_out, double* gpu_ms,
                      sd_snapshot** snap_out, char* err, size_t errlen);

/* No counterpart in the reference's `Engine`: the questions of `Decider::ask_all` in one forward
 * (its engine half, src/lib.rs:192-198, forwards each question from the prefix snapshot in turn).
 * ids holds n_seqs independent sequences back to back (lens[q] tokens each); each one continues
 * from `cache` (nullable) exactly as its own `sd_engine_forward` would, so the results match
 * that forward's, while the weights stream once for the whole batch.  rows index the
 * concatenation; hidden_out as in sd_engine_forward.  No snapshot is kept.  Limits: 1 to 32
 * sequences; prefix + all sequences <= SD_CONTEXT; either every sequence has <= 20 tokens or every
 * one has more (the reference's matmul kernel choice depends on the length, src/engine.rs:419). */
int sd_engine_forward_batch(sd_engine* e, const uint32_t* ids, const size_t* lens, size_t n_seqs, const size_t* rows,
                            size_t n_rows, const sd_snapshot* cache, int timed, float* hidden_out, double* gpu_ms,
                            char* err, size_t errlen);

/* No counterpart in the reference's `Engine`: the question half of `Decider::ask_all`
 * (src/lib.rs:192-198: every question forwarded from the prefix snapshot, then `Head::probs`,
 * src/head.rs:66-77) with the pointer head evaluated on the device in f64.  Question i is
 * q_ids[i][0..q_lens[i]); its option rows options[i][0..n_options[i]) index into it and its answer
 * row is its last token.  probs_out receives sum(n_options) probabilities, question by question.
 * Questions of one matmul class (<= 20 tokens, or longer) run as independent sequences of batched
 * forwards (at most 32 each).  gpu_ms (nullable) receives the device time of all batches when
 * `timed`, NaN otherwise.  cache is the prefix snapshot (nullable: no prefix). */
int sd_engine_ask_batch(sd_engine* e, const sd_head* h, const sd_snapshot* cache, size_t n_questions,
                        const uint32_t* const* q_ids, const size_t* q_lens, const size_t* const* options,
                        const size_t* n_options, const double* temperatures, int timed, double* probs_out,
                        double* gpu_ms, char* err, size_t errlen);

/* `Snapshot::len` (src/engine.rs:82): prefix + forwarded tokens. */
size_t sd_snapshot_len(const sd_snapshot* s);

/* Drop of `Snapshot`. */
void sd_snapshot_free(sd_snapshot* s);

/* `Engine::profile(ids)` (src/engine.rs:668-711): device ms per kernel label, slowest first.
 * Fills up to `cap` (label, ms) pairs; *n_out receives the number of labels.  Labels are static
 * strings owned by the library. */
int sd_engine_profile(sd_engine* e, const uint32_t* ids, size_t n, const char** labels, double* ms, size_t cap,
                      size_t* n_out, char* err, size_t errlen);

/* `Head::load(bytes)` (src/head.rs:25-52): head.safetensors, all tensors F32. */
int sd_head_load(const uint8_t* bytes, size_t len, sd_head** out, char* err, size_t errlen);
void sd_head_free(sd_head* h);

/* `Head::probs(hidden, d, temperature)` (src/head.rs:66-77): hidden = [options..., answer] rows;
 * probs_out receives n_rows - 1 option probabilities. */
int sd_head_probs(const sd_head* h, const float* hidden, size_t n_rows, size_t d, double temperature,
                  double* probs_out, char* err, size_t errlen);

/* The engine half of `Decider::run` (src/lib.rs:183-199) on token ids: one question is a single
 * forward of state ++ question.  Several questions, all longer than 20 tokens, at most 31 of them,
 * with state + questions within the 4096-token context, run as ONE forward of the state with every
 * question as a branch of it: each branch attends the state's rows and its own, and its delta rule
 * continues from the state's final state and conv history, which is what the reference computes
 * from the state's snapshot.  Otherwise the state runs once (keep = true) and the questions
 * continue from its snapshot (as sd_engine_ask_batch).  STRANDS_DECIDER_TREE=0 in the environment
 * turns the one-forward form off.  Either form leaves no snapshot behind; the live caches hold the
 * last forward's rows.  options[i][0..n_options[i]) are option token
 * indices into question i; probs_out receives sum(n_options) probabilities, question by question.
 * The head runs on the device (f64). */
int sd_ask_ids(sd_engine* e, const sd_head* h, const uint32_t* state, size_t n_state, size_t n_questions,
               const uint32_t* const* q_ids, const size_t* q_lens, const size_t* const* options,
               const size_t* n_options, const double* temperatures, double* probs_out, char* err, size_t errlen);

/* ---- kernel-level entry points on device buffers (per-configuration benchmarks and tests) ---- */

/* Y[M,N] f16 = A[M,K] f16 . deq(W)^T, W int4 group-32 symmetric in the model layout
 * ([N][K/32] blocks of 4 u32, scales [N][K/32] f16): the reference's matmul_gemv/matmul_tiled
 * (src/kernels.rs:590-709).  exact = 1 selects the GEMV's f32 dequant, 0 the tiled f16 dequant;
 * cfg < 0 takes the engine's choice for the shape (tile and split-K).  packed = 0: Wq and Sc are
 * in the model's order and layout and are rewritten into a library workspace on every call;
 * packed = 1: they were already rewritten by sd_op_repack_w4 (what the engine does to its weights
 * once at load). */
int sd_op_matmul(const void* A, const void* Wq, const void* Sc, void* Y, int M, int N, int K, int exact, int cfg,
                 int packed, void* stream, char* err, size_t errlen);

/* No counterpart in the reference: rewrites an N x K int4 matrix in place into what the GEMM
 * kernels read (sd_op_matmul with packed = 1): the N*K/8 words into the engine nibble order and,
 * when N is a multiple of 32 and K of 64, words and scales into 32-column x 64-k tiles (each tile's
 * blocks contiguous, column by column). */
int sd_op_repack_w4(void* Wq, void* Sc, int N, int K, void* stream, char* err, size_t errlen);

/* One gated-delta-net recurrence, the reference's Gdn kernel (src/kernels.rs:257-372), on device
 * buffers: qkv [L][2*H*dk + H*dv] f32, a/b gates f16 in big [L][stride] at a_off + h / b_off + h,
 * negA[H], dt_bias[H] f32; state [H][dk][dv] f32 (read when load_state, always written);
 * o [L][H*dv] f32. */
int sd_op_gdn(const void* qkv, const void* big, int stride, int a_off, int b_off, const void* negA, const void* dtb,
              int L, int H, int dk, int dv, void* state, int load_state, void* o, void* stream, char* err,
              size_t errlen);

/* No counterpart in the reference: sd_op_matmul (cfg < 0, packed = 1) for callers that cannot
 * allocate device memory, such as code under HIP graph capture or serving loops that forbid
 * hipMalloc.  It calls no hipMalloc, hipFree or other allocating routine: the split-K partial slots
 * go to a fixed 16 MiB device array of the library (one per GPU, held until the process ends).  The
 * weights must already be in what the kernels read (sd_op_repack_w4); f16 dequant (exact = 0) needs
 * N a multiple of 32.  The results are those of sd_op_matmul for the same arguments, except where
 * sd_op_matmul's split-K slots (ks * M * N f32) exceed the array (prefill shapes from about 520 rows
 * at K = 6144): those run with the largest split that fits, down to none, and their slot sums can
 * differ from sd_op_matmul's by one f16 rounding.  The array's device address is looked up on the
 * first call on a device: before capturing calls into a graph, make one call outside the capture.
 * Every call on one GPU shares that array: calls that overlap on one GPU (other streams, other
 * threads) race. */
int sd_op_matmul_noalloc(const void* A, const void* Wq, const void* Sc, void* Y, int M, int N, int K, int exact,
                         void* stream, char* err, size_t errlen);

/* The reference's matmul_gemv(f) (src/kernels.rs:590-635, decode 550-576) for any of its weight
 * formats, on device buffers in the model's layout: Y[M,N] f16 = A[M,K] f16 . deq(W)^T with W
 * [N][K/32] blocks of 4*bits bytes (int2/int3/int4), scales [N][K/group] f16 and, when asym, biases
 * Bi [N][K/group] f16; the weights are dequantized in f32 ((q - 2^(bits-1)) s, or fma(q, s, b)). */
int sd_op_matmul_fmt(const void* A, const void* Wq, const void* Sc, const void* Bi, void* Y, int M, int N, int K,
                     int bits, int group, int asym, void* stream, char* err, size_t errlen);

/* No counterpart in the reference: the split-K form of sd_op_matmul that the engine uses for the
 * projections feeding the residual add: part[z][M][N] f32 (z < ks) holds the partial product over
 * the z-th k range, whose slot-order sum rounded to f16 is Y.  exact = 1: the f32-dequant GEMV (cfg
 * ignored); else configuration cfg (0 <= cfg) with f16 dequant.  packed as in sd_op_matmul. */
int sd_op_matmul_split(const void* A, const void* Wq, const void* Sc, void* part, int M, int N, int K, int exact,
                       int cfg, int ks, int packed, void* stream, char* err, size_t errlen);

/* gate_up followed by silu_mul (src/kernels.rs:123-135, 590-709) as the engine fuses them:
 * mid[M][N/2] f16 = f16(silu(g) * u) with [g | u] = f16(A . deq(W)^T), W the model's gate_up ([gate
 * (N/2) | up (N/2)] rows, int4 g32).  exact = 1: the GEMV's f32 dequant, else the tiled f16 dequant
 * with configuration cfg (< 0: the engine's choice). */
int sd_op_gate_up_silu(const void* A, const void* Wq, const void* Sc, void* mid, int M, int N, int K, int exact, int cfg,
                       void* stream, char* err, size_t errlen);

/* embed (src/kernels.rs:63-89): x[L][d] f32 = the dequantized table rows ids[0..L) (u32), table Q
 * [vocab][d/32][bits] u32 words, scales S (and asym biases Bi) [vocab][d/group] f16. */
int sd_op_embed(const void* ids, int L, const void* Q, const void* S, const void* Bi, int d, int bits, int group, int asym,
                void* x, void* stream, char* err, size_t errlen);

/* add_norm (src/kernels.rs:93-120): for r < nrows, row = rows[r] (u32; rows null: r): x[row] += y[row]
 * (f16 [.][d], nullable: no add), then out[r] = x[row] rsqrt(mean(x[row]^2) + 1e-6) w as f16 (h16)
 * or f32 (h32); exactly one of h16, h32. */
int sd_op_add_norm(void* x, const void* y, const void* w, int d, const void* rows, int nrows, void* h16, void* h32,
                   void* stream, char* err, size_t errlen);

/* silu_mul (src/kernels.rs:123-135): mid[L][I] f16 = f16(silu(g) u), big[L] = [g (I) | u (I)] f16. */
int sd_op_silu_mul(const void* big, int L, int I, void* mid, void* stream, char* err, size_t errlen);

/* add_bias (src/kernels.rs:138-149): y[L][N] f16 += c[N] f32 (the adapter layers' bias). */
int sd_op_add_bias(void* y, int L, int N, const void* c, void* stream, char* err, size_t errlen);

/* conv (src/kernels.rs:152-170): out[t][c] f32 = silu(sum_j w[c][j] x[t + j - 3][c]) over channels
 * c < C of big [L][stride] f16, rows before 0 from hist [3][C] f16; w [C][4] f32. */
int sd_op_conv(const void* big, int stride, int L, int C, const void* w, const void* hist, void* out, void* stream,
               char* err, size_t errlen);

/* gnorm (src/kernels.rs:377-396): out[t][h*DV + c] f16 = f16(w[c] o rsqrt(mean_c(o^2) + 1e-6) silu(z)),
 * o [L][H*DV] f32, z = big[t*stride + z_off + h*DV + c] f16, w [DV] f32 (DV = 128). */
int sd_op_gnorm(const void* o, const void* big, int stride, int z_off, const void* w, int L, int H, int DV, void* out,
                void* stream, char* err, size_t errlen);

/* qk_prep then attn (src/kernels.rs:400-541) for one sequence at cache rows P .. P+L-1: Q [HQ][L][HD]
 * f16 receives the normed, rotated queries; the K cache Kc, in blocks of 32 rows [HK][ctx/32][HD/32]
 * [32 rows][32 dims], and the V cache Vt, transposed in blocks of 32 rows [HK][ctx/32][HD][32] (f16,
 * the engine's layouts), receive rows P .. P+L-1, rows below P are the prefix; out [L][HQ*HD] f16 the gated attention output.  big [L][stride]
 * holds [q | gate] per q head, then K, V heads; rope [ctx][RD/2][2] f32 (cos, sin).  head_dim 256
 * only, ctx a multiple of 32.  With RD 64 the attention normalizes and rotates the queries from big
 * itself (as the engine's forward does) and Q is written for the caller only. */
int sd_op_attention(const void* big, int stride, const void* qw, const void* kw, const void* rope, int L, int P, int HQ,
                    int HK, int HD, int RD, void* Q, void* Kc, void* Vt, int ctx, void* out, void* stream, char* err,
                    size_t errlen);

/* No counterpart in the reference (a test hook for per-layer parity): the forward of ids from cache
 * (nullable) run step by step; after every residual add + RMSNorm of the layers (each layer's
 * in_norm, then its post_norm) the residual x (f32) and the normalized h (f16 bits) of rows[0..n_rows)
 * are copied to x_out / h_out + tap * n_rows * hidden.  At most cap taps are copied; *n_taps receives
 * the number the forward has.  The live state afterwards is that of a forward without keep. */
int sd_engine_trace(sd_engine* e, const uint32_t* ids, size_t n, const sd_snapshot* cache, const size_t* rows,
                    size_t n_rows, float* x_out, uint16_t* h_out, size_t cap, size_t* n_taps, char* err, size_t errlen);

#ifdef __cplusplus
}
#endif

#endif /* SDHIP_H */
