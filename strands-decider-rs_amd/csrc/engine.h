// Engine state: the counterpart of the reference's `Engine`, `Pool`, `Plan` and `Snapshot`
// (src/engine.rs:57-132), laid out for one MI355X.
#pragma once

#include <functional>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/sdhip.h"
#include "common.h"
#include "head.h"

namespace sd {

struct TensorRef {
    uint64_t offset, bytes;
    uint32_t N, K, bits, group;
    bool asym;
};

struct Shard {
    uint64_t start = 0, bytes = 0;
    void* dev = nullptr;
};

struct Mat {
    const uint32_t* q = nullptr;
    const f16* s = nullptr;
    const f16* b = nullptr;  // asymmetric biases [N][K/group]
    int N = 0, K = 0;
    int bits = 4, group = 32;
    bool asym = false;
    bool tiled = false;  // int4 g32 symmetric, words and scales in the tiled layout (tile_w4)
    // the reference's default format: the only one its tiled matmul takes (src/engine.rs:434-442)
    bool deflt() const { return bits == 4 && group == 32 && !asym; }
};

struct EmbedW {
    const uint32_t* q = nullptr;
    const f16* s = nullptr;
    const f16* b = nullptr;
    int bits = 4, group = 32;
    bool asym = false;
};

struct LayerW {
    int kind = 0;
    const float* in_norm = nullptr;
    const float* post_norm = nullptr;
    Mat in_proj, out_proj, qkv, o_proj, gate_up, down, proj;
    const float *conv = nullptr, *negA = nullptr, *dtb = nullptr, *gnorm = nullptr;
    const float *q_norm = nullptr, *k_norm = nullptr, *bias = nullptr;
    float* state = nullptr;  // [H][dk][dv] f32 (in the live arena)
    f16* hist = nullptr;     // [3][C] f16 (in the live arena)
    size_t state_off = 0, hist_off = 0;  // their byte offsets in an arena image (live or a snapshot's)
    f16* kc = nullptr;       // [hk][CONTEXT][hd] f16
    f16* vc = nullptr;       // [hk][hd][CONTEXT] f16 (transposed for the attention kernel)
};

struct Cfg {
    int d = 0, inter = 0, hq = 0, hk = 0, hd = 0, rd = 0, H = 0, dk = 0, dv = 0;
    double theta = 0;
};

// Activation buffers for up to `cap` tokens, shared by every plan (src/engine.rs:62-78).
struct Pool {
    int cap = 0;
    void* base = nullptr;
    // Everything the host sends before a forward sits in one block at the start of the pool (the
    // lu block, ids, rows, the Segs tables), mirrored by a pinned host block: one copy per forward.
    size_t up_bytes = 0, off_ids = 0, off_rows = 0, off_seg_row = 0, off_seg_chunk = 0, off_seg_seq = 0;
    uint32_t *ids = nullptr, *rows = nullptr;
    float *x = nullptr, *qkvc = nullptr, *of = nullptr, *out = nullptr;
    // a compact last layer's rows: the read rows of the residual stream and of the mixer output
    float* xc = nullptr;
    f16* oc = nullptr;
    f16 *h = nullptr, *big = nullptr, *mid = nullptr, *o = nullptr, *y = nullptr, *q = nullptr;
    GdnWs gdn;
    float* attn_ws = nullptr;
    int attn_rows = 0;
    float* ypart = nullptr;  // split-K partials of the projections that feed the residual add
    size_t ypart_elems = 0;
    float* gpart = nullptr;  // split-K partials of gate_up (summed by silu * mul)
    size_t gpart_elems = 0;
    uint32_t *seg_row = nullptr, *seg_chunk = nullptr, *seg_seq = nullptr;  // Segs tables
    int seg_chunk_cap = 0;
};

struct Step {
    const char* label;
    std::function<void(hipStream_t)> run;
};

// The dispatch list for one token length and its captured graph (src/engine.rs:57-60, 396-524).
struct Plan {
    int L = 0;
    std::vector<Step> steps;
    YIn last_y;  // where the last sublayer output lives (read by the final norm)
    int compact = 0;  // > 0: the last layer's tail ran on this many read rows (compact, in pool.xc)
    uint64_t used = 0;  // Engine::plan_clock at the last use (least recently used plans are evicted)
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    void destroy();
};

struct Engine;

// Prefix state after a forward: GDN state + conv history (the live arena image), then compact
// K [hk][len][hd] and V [hk][hd][len] per attention layer (src/engine.rs:81-87, 592-614).
struct Snapshot {
    const Engine* engine = nullptr;
    size_t len = 0;
    uint64_t id = 0;
    void* arena = nullptr;  // [arena image | per attention layer: K, V^T blocks of the first len32 keys per kv head]
    size_t alloc_bytes = 0;
    size_t arena_bytes = 0, kv_stride = 0;  // kv_stride: hk * len32 * hd * 2, len32 = len rounded up to 32
    uint8_t* kv(size_t attn_index, int which) const {
        return static_cast<uint8_t*>(arena) + arena_bytes + (attn_index * 2 + which) * kv_stride;
    }
    ~Snapshot();
};

struct Engine {
    Cfg cfg;
    std::vector<int> kinds;
    std::vector<double> unrotate;
    std::string adapter;
    hipStream_t st = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    std::unordered_map<std::string, TensorRef> tensors;
    std::vector<Shard> shards;
    std::unordered_map<std::string, void*> embed_parts;
    EmbedW emb;
    int vocab = 0;
    std::vector<LayerW> layers;
    std::vector<int> attn_layers;
    const float* final_norm = nullptr;
    float* rope = nullptr;
    uint32_t* lu = nullptr;  // device [L, P, CONTEXT, has_cache, chunks, sequences, 0, 0] (start of the pool)
    uint8_t* up_h = nullptr;  // host mirror of the pool's upload block
    size_t up_h_bytes = 0, up_dirty = 0;
    uint8_t* arena = nullptr;  // [GDN states | conv histories]
    size_t arena_bytes = 0, arena_state_bytes = 0;
    int n_linear = 0;
    int max_n = 0;
    uint64_t snapshot_ids = 0, kv_owner = 0;
    // Freed snapshot buffers kept for reuse (a snapshot is made by every keep-forward; hipMalloc and
    // hipFree would each cost more than its copies).  A snapshot may be freed from another thread.
    mutable std::mutex snap_mu;
    mutable std::vector<std::pair<void*, size_t>> snap_pool;
    void* snap_alloc(size_t bytes);
    void snap_release(void* p, size_t bytes) const;
    bool use_graphs = true;
    // STRANDS_DECIDER_CHECKED=1 (the reference's switch for shader runtime checks, src/engine.rs:283,
    // 335-338): every step runs eagerly and is synchronized, a GPU error names the step that raised
    // it, and the residual stream is checked for non-finite values after every add + RMSNorm.
    bool checked = false;
    void run_checked(Plan& pl);
    bool gu_il = false;  // gate_up weights interleaved in groups of 16 rows (interleave_gate_up)
    Pool pool;
    std::map<uint64_t, Plan> plans;
    uint64_t plan_clock = 0;
    // Captured plans kept at most: each holds an instantiated graph of ~230 kernel nodes (the pool's
    // buffers are shared, so a plan costs no activation memory of its own).  Traffic with more
    // distinct (length, sequences) keys evicts the least recently used one; the configs[4] sweep
    // (64 state lengths and 64 question batches) stays cached.
    static constexpr size_t kMaxPlans = 512;
    float* out_h = nullptr;
    int out_h_cap = 0;
    std::vector<void*> device_allocs, host_allocs;
    // Device copy of the last head used by ask_batch, and the head's per-call buffers.
    HeadW headw;
    uint64_t head_id = 0;
    void* head_dev = nullptr;     // the head's weights
    double* unrot_dev = nullptr;  // `unrotate` on the device (rotated torsos only)
    // Per-call buffers of ask_batch for up to `rows` rows / `nq` questions: device [proj | scale |
    // probs | qtab | ooff | is_answer], pinned host [scale | probs | qtab | ooff | is_answer].
    struct HeadBufs {
        size_t rows = 0, nq = 0, dim = 0;
        void *dev = nullptr, *host = nullptr;
        double *proj = nullptr, *scale = nullptr, *probs = nullptr;
        uint32_t *qtab = nullptr, *ooff = nullptr;
        uint8_t* is_answer = nullptr;
        double *scale_h = nullptr, *probs_h = nullptr;
        uint32_t *qtab_h = nullptr, *ooff_h = nullptr;
        uint8_t* is_answer_h = nullptr;
    } hb;
    void ensure_head_bufs(size_t rows, size_t nq);

    ~Engine();
    void load(const sd_config* c, const sd_tensor* ts, size_t nt, const char* const* shard_paths,
              const uint64_t* shard_starts, const uint64_t* shard_bytes, size_t ns, const sd_embed* em);
    void forward(const uint32_t* ids, size_t n, const size_t* rows, size_t n_rows, const Snapshot* cache, bool keep,
                 bool timed, float* hidden, double* gpu_ms, Snapshot** snap_out);
    // Several independent sequences (ids = their concatenation, lens[q] tokens each) in one
    // forward, each continuing from `cache` (nullable) as its own forward would; rows index the
    // concatenation.  No snapshot.  Every sequence must be <= 20 tokens, or every one longer (the
    // reference's matmul choice depends on the length).
    void forward_batch(const uint32_t* ids, const size_t* lens, size_t nseq, const size_t* rows, size_t n_rows,
                       const Snapshot* cache, bool timed, float* hidden, double* gpu_ms);
    // forward_batch followed by the pointer head on the device: sequence q's rows are n_opts[q]
    // option rows then its answer row (rows lists them sequence by sequence); probs receives
    // sum(n_opts) option probabilities, sequence by sequence.  gpu_ms covers torso and head.
    void ask_batch(const Head& head, const uint32_t* ids, const size_t* lens, size_t nseq, const size_t* rows,
                   const size_t* n_opts, const double* temps, const Snapshot* cache, bool timed, double* probs,
                   double* gpu_ms);
    // Decider::ask_all's engine half (src/lib.rs:192-198) in one forward: the state (n_state rows)
    // and the questions (lens[q] rows each, > 20 tokens: the tiled matmuls' f16 dequant, as their
    // own forwards use) as branches that continue from it.  The weights stream once for all rows.
    // Each question's hidden rows and probabilities are those of its forward from the state's
    // snapshot (within the parity tolerances: the matmul tiles differ with the row count).  rows,
    // n_opts, temps, probs and gpu_ms as in ask_batch; rows index the questions' concatenation.
    // No snapshot is kept.
    void ask_tree(const Head& head, const uint32_t* state, size_t n_state, const uint32_t* ids, const size_t* lens,
                  size_t nq, const size_t* rows, const size_t* n_opts, const double* temps, bool timed, double* probs,
                  double* gpu_ms);
    std::vector<std::pair<const char*, double>> profile(const uint32_t* ids, size_t n);
    // The forward of `ids` from `cache` run step by step, copying after every residual add + RMSNorm
    // of the layers (each layer's in_norm, then its post_norm) the residual x (f32) and the
    // normalized h (f16 bits) of the given rows: tap i goes to x_out / h_out + i * n_rows * d.  At
    // most `cap` taps are copied; returns the number the plan has.  A test hook for per-layer parity.
    size_t trace(const uint32_t* ids, size_t n, const Snapshot* cache, const size_t* rows, size_t n_rows, float* x_out,
                 uint16_t* h_out, size_t cap);

   private:
    void* dalloc(size_t bytes);
    void* halloc(size_t bytes);
    const TensorRef& tensor(const std::string& name) const;
    const void* dptr(const std::string& name) const;
    Mat mat(const std::string& name) const;
    const float* f32(const std::string& name, size_t count) const;
    void ensure_pool(int l);
    // The plan for L rows: one sequence (nseq = 0) or nseq independent ones; short: the reference's
    // GEMV dequant (each sequence <= 20 tokens).
    // tree > 0: sequence 0 is a state of `tree` rows and sequences 1 .. nseq - 1 continue from it
    // (their own rows attend to its rows, their delta rule starts from its final state), each as its
    // own forward from the state's snapshot would; see ask_tree.
    Plan& plan(int L, int nseq = 0, bool short_seqs = false, int tree = 0, bool cache_only = false, int rows_read = 0);
    void upload(const uint32_t* ids, size_t n, const size_t* rows, size_t n_rows, size_t P, bool has_cache,
                uint32_t chunks, uint32_t nseq, const Snapshot* cache, uint32_t tree = 0);
    void restore(const Snapshot* cache, size_t P);
    void launch_and_read(Plan& pl, size_t n_rows, bool timed, bool read = true);
    // Validation, sequence tables, upload and restore of a batched forward; returns its plan.
    Plan& prepare_batch(const uint32_t* ids, const size_t* lens, size_t nseq, const size_t* rows, size_t n_rows,
                        const Snapshot* cache);
    void attach_head(const Head& head);
    // The common tail of ask_batch and ask_tree: the head tables, the forward, the device head.
    void ask_tail(Plan& pl, size_t nseq, const size_t* n_opts, const double* temps, size_t n_rows, size_t n_prob,
                  bool timed, double* probs, double* gpu_ms);
    void finish(size_t n_rows, float* hidden, bool timed, double* gpu_ms);
    void mm(std::vector<Step>& steps, const char* label, const f16* A, const Mat& m, f16* Y, int L, bool short_rows);
    YIn mm_y(std::vector<Step>& steps, const char* label, const f16* A, const Mat& m, int L, bool short_rows);
};

}  // namespace sd
