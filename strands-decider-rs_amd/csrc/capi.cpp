// extern "C" entry points declared in include/sdhip.h.  Every call catches C++ exceptions and
// reports them through (err, errlen), the C form of the reference's `crate::Error(String)`.
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>

#include "engine.h"
#include "head.h"

namespace {

void put_err(char* err, size_t errlen, const char* msg) {
    if (!err || errlen == 0) return;
    std::strncpy(err, msg, errlen - 1);
    err[errlen - 1] = '\0';
}

template <class F>
int guarded(char* err, size_t errlen, F&& f) {
    try {
        f();
        if (err && errlen) err[0] = '\0';
        return 0;
    } catch (const std::exception& e) {
        put_err(err, errlen, e.what());
    } catch (...) {
        put_err(err, errlen, "unknown error");
    }
    return 1;
}

sd::Engine* E(sd_engine* e) { return reinterpret_cast<sd::Engine*>(e); }
const sd::Engine* E(const sd_engine* e) { return reinterpret_cast<const sd::Engine*>(e); }
sd::Snapshot* S(sd_snapshot* s) { return reinterpret_cast<sd::Snapshot*>(s); }
const sd::Snapshot* S(const sd_snapshot* s) { return reinterpret_cast<const sd::Snapshot*>(s); }
const sd::Head* Hd(const sd_head* h) { return reinterpret_cast<const sd::Head*>(h); }

// Device workspace for the kernel-level entry points (grown on demand, kept until exit).
struct OpWs {
    std::mutex mu;
    float* part = nullptr;
    size_t part_floats = 0;
    void* gdn = nullptr;
    size_t gdn_bytes = 0;
    // the weights and scales of sd_op_matmul in the engine's order and layout, and the scratch of
    // the tiled-layout rewrite
    void* wpack = nullptr;
    size_t wpack_bytes = 0;
    void* wtmp = nullptr;
    size_t wtmp_bytes = 0;
    void* attn = nullptr;  // sd_op_attention: the lu block, then the key-split workspace
    size_t attn_bytes = 0;
};
void grow(void*& p, size_t& have, size_t need) {
    if (have >= need) return;
    if (p) SD_HIP(hipFree(p));
    p = nullptr;
    have = 0;
    SD_HIP(hipMalloc(&p, need));
    have = need;
}
OpWs& op_ws() {
    static OpWs w;
    return w;
}

}  // namespace

namespace {

// The weights of an int4 g32 matrix in what the kernels read: the caller's own when already
// rewritten by sd_op_repack_w4 (packed) or when the shape keeps the model's layout (the GEMV's),
// else a rewritten copy in the workspace (engine nibble order, tiled).  `force_engine_order`: the
// kernel wants the engine nibble order even where the shape is not tileable (the f16-dequant
// configurations).
std::pair<const uint32_t*, const sd::f16*> op_weights(OpWs& w, const void* Wq, const void* Sc, int N, int K, bool packed,
                                                      bool force_engine_order, hipStream_t st) {
    const bool tiled = sd::w4_tileable(N, K);
    if ((packed && tiled) || (!tiled && !force_engine_order))
        return {static_cast<const uint32_t*>(Wq), static_cast<const sd::f16*>(Sc)};
    const size_t words = (size_t)N * K / 8, scales = (size_t)N * K / 32;
    grow(w.wpack, w.wpack_bytes, words * 4 + scales * 2);
    auto* pw = static_cast<uint32_t*>(w.wpack);
    auto* ps = reinterpret_cast<sd::f16*>(pw + words);
    SD_HIP(hipMemcpyAsync(pw, Wq, words * 4, hipMemcpyDeviceToDevice, st));
    SD_HIP(hipMemcpyAsync(ps, Sc, scales * 2, hipMemcpyDeviceToDevice, st));
    sd::repack_w4(pw, words, st);
    if (tiled) {
        grow(w.wtmp, w.wtmp_bytes, words * 4 + scales * 2);
        sd::tile_w4(pw, ps, N, K, w.wtmp, st);
    }
    return {pw, ps};
}

}  // namespace

extern "C" {

int sd_engine_load(const sd_config* cfg, const sd_tensor* tensors, size_t n_tensors, const char* const* shard_paths,
                   const uint64_t* shard_starts, const uint64_t* shard_bytes, size_t n_shards, const sd_embed* embed,
                   sd_engine** out, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!out) throw sd::Error("sd_engine_load: null output");
        auto e = std::make_unique<sd::Engine>();
        e->load(cfg, tensors, n_tensors, shard_paths, shard_starts, shard_bytes, n_shards, embed);
        *out = reinterpret_cast<sd_engine*>(e.release());
    });
}

void sd_engine_free(sd_engine* e) { delete E(e); }

size_t sd_engine_hidden_size(const sd_engine* e) { return e ? (size_t)E(e)->cfg.d : 0; }

const char* sd_engine_adapter(const sd_engine* e) { return e ? E(e)->adapter.c_str() : ""; }

int sd_engine_forward(sd_engine* e, const uint32_t* ids, size_t n, const size_t* rows, size_t n_rows,
                      const sd_snapshot* cache, int keep, int timed, float* hidden_out, double* gpu_ms,
                      sd_snapshot** snap_out, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!e || (!ids && n) || (!rows && n_rows) || (!hidden_out && n_rows)) throw sd::Error("sd_engine_forward: null argument");
        if (keep && !snap_out) throw sd::Error("sd_engine_forward: keep needs snap_out");
        sd::Snapshot* snap = nullptr;
        E(e)->forward(ids, n, rows, n_rows, S(cache), keep != 0, timed != 0, hidden_out, gpu_ms, keep ? &snap : nullptr);
        if (snap_out) *snap_out = reinterpret_cast<sd_snapshot*>(snap);
    });
}

int sd_engine_forward_batch(sd_engine* e, const uint32_t* ids, const size_t* lens, size_t n_seqs, const size_t* rows,
                            size_t n_rows, const sd_snapshot* cache, int timed, float* hidden_out, double* gpu_ms,
                            char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!e || !ids || !lens || (!rows && n_rows) || (!hidden_out && n_rows))
            throw sd::Error("sd_engine_forward_batch: null argument");
        E(e)->forward_batch(ids, lens, n_seqs, rows, n_rows, S(cache), timed != 0, hidden_out, gpu_ms);
    });
}

size_t sd_snapshot_len(const sd_snapshot* s) { return s ? S(s)->len : 0; }

void sd_snapshot_free(sd_snapshot* s) { delete S(s); }

int sd_engine_profile(sd_engine* e, const uint32_t* ids, size_t n, const char** labels, double* ms, size_t cap,
                      size_t* n_out, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!e || !ids) throw sd::Error("sd_engine_profile: null argument");
        const auto by = E(e)->profile(ids, n);
        for (size_t i = 0; i < by.size() && i < cap; i++) {
            labels[i] = by[i].first;
            ms[i] = by[i].second;
        }
        if (n_out) *n_out = by.size();
    });
}

int sd_head_load(const uint8_t* bytes, size_t len, sd_head** out, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!bytes || !out) throw sd::Error("sd_head_load: null argument");
        auto h = std::make_unique<sd::Head>();
        h->load(bytes, len);
        *out = reinterpret_cast<sd_head*>(h.release());
    });
}

void sd_head_free(sd_head* h) { delete reinterpret_cast<sd::Head*>(h); }

int sd_head_probs(const sd_head* h, const float* hidden, size_t n_rows, size_t d, double temperature,
                  double* probs_out, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!h || !hidden || !probs_out) throw sd::Error("sd_head_probs: null argument");
        const auto p = Hd(h)->probs(hidden, n_rows, d, temperature);
        std::memcpy(probs_out, p.data(), p.size() * sizeof(double));
    });
}

namespace {

// STRANDS_DECIDER_TREE=0 turns the one-forward ask_all off (the snapshot path then serves every call).
bool tree_ask_enabled() {
    static const bool on = [] {
        const char* v = std::getenv("STRANDS_DECIDER_TREE");
        return !(v && std::strcmp(v, "0") == 0);
    }();
    return on;
}

// The questions of an ask_all, each continuing from `prefix` (src/lib.rs:192-198), with the pointer
// head on the device.  They run as independent sequences of batched forwards (the same results as
// one forward each; the weights stream once per batch).  A batch holds questions of one matmul
// class (<= 20 tokens or longer, src/engine.rs:419) and fits the context after the prefix.
void ask_from(sd::Engine* eng, const sd::Head& head, const sd::Snapshot* prefix, size_t n_questions,
              const uint32_t* const* q_ids, const size_t* q_lens, const size_t* const* options, const size_t* n_options,
              const double* temperatures, bool timed, double* probs_out, double* gpu_ms) {
    const size_t P = prefix ? prefix->len : 0;
    std::vector<std::vector<size_t>> batches;
    for (int cls = 0; cls < 2; cls++) {
        std::vector<size_t> cur;
        size_t tokens = 0;
        for (size_t i = 0; i < n_questions; i++) {
            if ((q_lens[i] <= 20) != (cls == 0)) continue;
            if (!cur.empty() && (cur.size() == (size_t)sd::SD_MAX_SEQS || P + tokens + q_lens[i] > SD_CONTEXT)) {
                batches.push_back(cur);
                cur.clear();
                tokens = 0;
            }
            cur.push_back(i);
            tokens += q_lens[i];
        }
        if (!cur.empty()) batches.push_back(cur);
    }
    std::vector<size_t> out_at(n_questions);  // where question i's probabilities go
    for (size_t i = 0, o = 0; i < n_questions; i++) {
        out_at[i] = o;
        o += n_options[i];
    }
    double total_ms = 0.0;
    for (const auto& b : batches) {
        std::vector<uint32_t> ids;
        std::vector<size_t> lens, rows, nopt;
        std::vector<double> temps;
        size_t np = 0;
        for (size_t i : b) {
            const size_t base = ids.size();
            for (size_t k = 0; k < n_options[i]; k++) rows.push_back(base + options[i][k]);
            rows.push_back(base + q_lens[i] - 1);
            ids.insert(ids.end(), q_ids[i], q_ids[i] + q_lens[i]);
            lens.push_back(q_lens[i]);
            nopt.push_back(n_options[i]);
            temps.push_back(temperatures[i]);
            np += n_options[i];
        }
        std::vector<double> p(np);
        double ms = 0.0;
        eng->ask_batch(head, ids.data(), lens.data(), lens.size(), rows.data(), nopt.data(), temps.data(), prefix,
                       timed, p.data(), &ms);
        total_ms += ms;
        size_t o = 0;
        for (size_t i : b) {
            std::memcpy(probs_out + out_at[i], p.data() + o, n_options[i] * sizeof(double));
            o += n_options[i];
        }
    }
    if (gpu_ms) *gpu_ms = timed ? total_ms : NAN;
}

void check_questions(size_t n_questions, const uint32_t* const* q_ids, const size_t* q_lens,
                     const size_t* const* options, const size_t* n_options, const double* temperatures) {
    if (n_questions == 0) throw sd::Error("ask at least one question");
    if (!q_ids || !q_lens || !options || !n_options || !temperatures) throw sd::Error("null question argument");
    for (size_t i = 0; i < n_questions; i++) {
        if (q_lens[i] == 0 || !q_ids[i]) throw sd::Error("question " + std::to_string(i) + " has no tokens");
        if (n_options[i] == 0 || !options[i]) throw sd::Error("question " + std::to_string(i) + " has no options");
        for (size_t k = 0; k < n_options[i]; k++)
            if (options[i][k] >= q_lens[i])
                throw sd::Error("question " + std::to_string(i) + ": option row " + std::to_string(options[i][k]) +
                                " out of range for " + std::to_string(q_lens[i]) + " tokens");
    }
}

}  // namespace

int sd_engine_ask_batch(sd_engine* e, const sd_head* h, const sd_snapshot* cache, size_t n_questions,
                        const uint32_t* const* q_ids, const size_t* q_lens, const size_t* const* options,
                        const size_t* n_options, const double* temperatures, int timed, double* probs_out,
                        double* gpu_ms, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!e || !h || !probs_out) throw sd::Error("sd_engine_ask_batch: null argument");
        check_questions(n_questions, q_ids, q_lens, options, n_options, temperatures);
        ask_from(E(e), *Hd(h), S(cache), n_questions, q_ids, q_lens, options, n_options, temperatures, timed != 0,
                 probs_out, gpu_ms);
    });
}

int sd_ask_ids(sd_engine* e, const sd_head* h, const uint32_t* state, size_t n_state, size_t n_questions,
               const uint32_t* const* q_ids, const size_t* q_lens, const size_t* const* options,
               const size_t* n_options, const double* temperatures, double* probs_out, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!e || !h || !probs_out || (!state && n_state)) throw sd::Error("sd_ask_ids: null argument");
        check_questions(n_questions, q_ids, q_lens, options, n_options, temperatures);
        sd::Engine* eng = E(e);
        if (n_questions == 1) {
            // src/lib.rs:185-190: one forward of state ++ question.
            std::vector<uint32_t> ids(state, state + n_state);
            ids.insert(ids.end(), q_ids[0], q_ids[0] + q_lens[0]);
            std::vector<size_t> rows;
            for (size_t k = 0; k < n_options[0]; k++) rows.push_back(n_state + options[0][k]);
            rows.push_back(ids.size() - 1);
            const size_t len = ids.size();
            eng->ask_batch(*Hd(h), ids.data(), &len, 1, rows.data(), n_options, temperatures, nullptr, false,
                           probs_out, nullptr);
            return;
        }
        // src/lib.rs:192-198: the state once, every question continuing from it.
        if (n_state == 0) throw sd::Error("context of 0 tokens: must be 1 to " + std::to_string(SD_CONTEXT));
        // One forward holds the state and every question as branches of it when the questions are
        // all longer than 20 tokens (their matmuls are then the tiled kernels', as in their own
        // forwards) and state + questions fit the context; otherwise the state's snapshot, then the
        // questions from it in batched forwards.
        bool tree = n_questions + 1 <= (size_t)sd::SD_MAX_SEQS && tree_ask_enabled();
        size_t total = n_state;
        for (size_t i = 0; i < n_questions; i++) {
            tree = tree && q_lens[i] > 20;
            total += q_lens[i];
        }
        if (tree && total <= SD_CONTEXT) {
            std::vector<uint32_t> ids;
            std::vector<size_t> rows;
            for (size_t i = 0; i < n_questions; i++) {
                const size_t base = ids.size();
                for (size_t k = 0; k < n_options[i]; k++) rows.push_back(base + options[i][k]);
                rows.push_back(base + q_lens[i] - 1);
                ids.insert(ids.end(), q_ids[i], q_ids[i] + q_lens[i]);
            }
            eng->ask_tree(*Hd(h), state, n_state, ids.data(), q_lens, n_questions, rows.data(), n_options,
                          temperatures, false, probs_out, nullptr);
            return;
        }
        sd::Snapshot* prefix = nullptr;
        eng->forward(state, n_state, nullptr, 0, nullptr, true, false, nullptr, nullptr, &prefix);
        std::unique_ptr<sd::Snapshot> hold(prefix);
        ask_from(eng, *Hd(h), prefix, n_questions, q_ids, q_lens, options, n_options, temperatures, false, probs_out,
                 nullptr);
    });
}

int sd_op_repack_w4(void* Wq, void* Sc, int N, int K, void* stream, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!Wq || !Sc) throw sd::Error("sd_op_repack_w4: null argument");
        if (N < 1 || K < 32 || K % 32) throw sd::Error("sd_op_repack_w4: need N >= 1 and K a multiple of 32");
        // other shapes keep the model's layout, which is what the GEMV reads for them
        if (!sd::w4_tileable(N, K)) return;
        const hipStream_t st = static_cast<hipStream_t>(stream);
        sd::repack_w4(static_cast<uint32_t*>(Wq), (size_t)N * K / 8, st);
        OpWs& w = op_ws();
        std::lock_guard<std::mutex> lock(w.mu);
        grow(w.wtmp, w.wtmp_bytes, (size_t)N * K / 2 + (size_t)N * K / 16);
        sd::tile_w4(static_cast<uint32_t*>(Wq), static_cast<sd::f16*>(Sc), N, K, w.wtmp, st);
    });
}

int sd_op_matmul(const void* A, const void* Wq, const void* Sc, void* Y, int M, int N, int K, int exact, int cfg,
                 int packed, void* stream, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!A || !Wq || !Sc || !Y) throw sd::Error("sd_op_matmul: null argument");
        if (cfg >= sd::gemm_w4_configs()) throw sd::Error("sd_op_matmul: no configuration " + std::to_string(cfg));
        if (M < 1 || N < 1 || K < 128 || K % 128) throw sd::Error("sd_op_matmul: need M, N >= 1 and K a multiple of 128");
        OpWs& w = op_ws();
        std::lock_guard<std::mutex> lock(w.mu);
        const hipStream_t st = static_cast<hipStream_t>(stream);
        if (exact && cfg < 0) {
            // the engine's choice for the GEMV rows: the f32-dequant GEMV, tiled where the shape is
            const auto wts = op_weights(w, Wq, Sc, N, K, packed != 0, false, st);
            const bool tiled = sd::w4_tileable(N, K);
            sd::gemv(static_cast<const sd::f16*>(A), wts.first, wts.second, nullptr, Y, 0, M, N, K, 4, 32, false, tiled,
                     sd::gemv_plan(M, N, K, tiled, 0, 0), st);
            return;
        }
        // cfg < 0: the engine's own choice for this shape (tile and split-K, the split summed by
        // reduce_partials here); cfg >= 0: that configuration, split until the grid covers the chip.
        const size_t cap = size_t(64) << 20;
        int c = cfg, ks = 1;
        if (cfg < 0) {
            const sd::GemmPlan p = sd::gemm_w4_plan(M, N, K, exact != 0, true, cap);
            c = p.cfg;
            ks = p.ks;
        } else {
            ks = sd::gemm_w4_split(M, N, K, c, 256, cap);
        }
        const auto* a = static_cast<const sd::f16*>(A);
        // The kernels read the engine nibble order and, where the shape has one, the tiled layout:
        // unless the caller rewrote its weights already (sd_op_repack_w4), rewrite a copy of them.
        const bool tiled = sd::w4_tileable(N, K);
        const auto wts = op_weights(w, Wq, Sc, N, K, packed != 0, true, st);
        const uint32_t* wq = wts.first;
        const sd::f16* sc = wts.second;
        if (ks == 1) {
            sd::gemm_w4(a, wq, sc, static_cast<sd::f16*>(Y), nullptr, M, N, K, exact != 0, 1, st, c, tiled);
            return;
        }
        if (w.part_floats < (size_t)ks * M * N) {
            if (w.part) SD_HIP(hipFree(w.part));
            w.part = nullptr;
            SD_HIP(hipMalloc(&w.part, cap * 4));
            w.part_floats = cap;
        }
        sd::gemm_w4(a, wq, sc, nullptr, w.part, M, N, K, exact != 0, ks, st, c, tiled);
        sd::reduce_partials(w.part, ks, (size_t)M * N, static_cast<sd::f16*>(Y), st);
    });
}

int sd_op_gdn(const void* qkv, const void* big, int stride, int a_off, int b_off, const void* negA, const void* dtb,
              int L, int H, int dk, int dv, void* state, int load_state, void* o, void* stream, char* err,
              size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!qkv || !big || !negA || !dtb || !state || !o) throw sd::Error("sd_op_gdn: null argument");
        if (L < 1 || L > SD_CONTEXT) throw sd::Error("sd_op_gdn: L must be 1 to 4096");
        if (dk != 128 || dv != 128) throw sd::Error("sd_op_gdn: only 128-wide key/value heads are supported");
        const sd::GdnShape s{H, dk, dv, stride, a_off, b_off, 0, 2 * H * dk + H * dv};
        OpWs& w = op_ws();
        std::lock_guard<std::mutex> lock(w.mu);
        const size_t need = sd::gdn_ws_bytes(L, s);
        if (need > w.gdn_bytes) {
            if (w.gdn) SD_HIP(hipFree(w.gdn));
            w.gdn = nullptr;
            SD_HIP(hipMalloc(&w.gdn, need));
            w.gdn_bytes = need;
        }
        sd::GdnWs ws;
        sd::gdn_ws_carve(w.gdn, L, s, ws);
        const hipStream_t st = static_cast<hipStream_t>(stream);
        sd::gdn_prep(static_cast<const float*>(qkv), static_cast<const sd::f16*>(big), s, static_cast<const float*>(negA),
                     static_cast<const float*>(dtb), L, ws, sd::ConvIn{}, sd::Segs{}, 0, nullptr, st);
        sd::gdn_scan(s, L, ws, static_cast<float*>(state), nullptr, load_state, static_cast<float*>(o), sd::Segs{}, 1, st);
    });
}

int sd_decode_scale_codes(const uint8_t* src, size_t src_bytes, size_t n, size_t g, uint16_t* dst, size_t dst_count,
                          char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!src || !dst) throw sd::Error("sd_decode_scale_codes: null argument");
        if (g == 0 || n > SIZE_MAX / (4 + g)) throw sd::Error("sd_decode_scale_codes: bad row shape");
        if (src_bytes < n * (4 + g))
            throw sd::Error("sd_decode_scale_codes: " + std::to_string(n) + " rows of " + std::to_string(g) +
                            " codes need " + std::to_string(n * (4 + g)) + " source bytes, got " + std::to_string(src_bytes));
        if (dst_count < n * g) throw sd::Error("sd_decode_scale_codes: the destination holds fewer than n * g scales");
        std::vector<double> pw;  // for this call only
        sd::decode_scale_codes(src, n, g, dst, pw);
    });
}

int sd_op_matmul_fmt(const void* A, const void* Wq, const void* Sc, const void* Bi, void* Y, int M, int N, int K,
                     int bits, int group, int asym, void* stream, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!A || !Wq || !Sc || !Y || (asym && !Bi)) throw sd::Error("sd_op_matmul_fmt: null argument");
        sd::gemv(static_cast<const sd::f16*>(A), static_cast<const uint32_t*>(Wq), static_cast<const sd::f16*>(Sc),
                 static_cast<const sd::f16*>(Bi), Y, 0, M, N, K, bits, group, asym != 0, false,
                 sd::gemv_plan(M, N, K, false, 0, 0), static_cast<hipStream_t>(stream));
    });
}

int sd_op_matmul_split(const void* A, const void* Wq, const void* Sc, void* part, int M, int N, int K, int exact,
                       int cfg, int ks, int packed, void* stream, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!A || !Wq || !Sc || !part) throw sd::Error("sd_op_matmul_split: null argument");
        if (M < 1 || N < 1 || K < 128 || K % 128) throw sd::Error("sd_op_matmul_split: need M, N >= 1 and K a multiple of 128");
        if (ks < 1 || ks > 8) throw sd::Error("sd_op_matmul_split: ks must be 1 to 8");
        OpWs& w = op_ws();
        std::lock_guard<std::mutex> lock(w.mu);
        const hipStream_t st = static_cast<hipStream_t>(stream);
        const bool tiled = sd::w4_tileable(N, K);
        const auto* a = static_cast<const sd::f16*>(A);
        if (exact) {
            const auto wts = op_weights(w, Wq, Sc, N, K, packed != 0, false, st);
            sd::GemvPlan p = sd::gemv_plan(M, N, K, tiled, 1, (size_t)ks * M * N);
            p.ks = ks;
            sd::gemv(a, wts.first, wts.second, nullptr, part, 1, M, N, K, 4, 32, false, tiled, p, st);
            return;
        }
        if (cfg < 0 || cfg >= sd::gemm_w4_configs()) throw sd::Error("sd_op_matmul_split: no configuration " + std::to_string(cfg));
        const auto wts = op_weights(w, Wq, Sc, N, K, packed != 0, true, st);
        sd::gemm_w4(a, wts.first, wts.second, nullptr, static_cast<float*>(part), M, N, K, false, ks, st, cfg, tiled);
    });
}

int sd_op_gate_up_silu(const void* A, const void* Wq, const void* Sc, void* mid, int M, int N, int K, int exact, int cfg,
                       void* stream, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!A || !Wq || !Sc || !mid) throw sd::Error("sd_op_gate_up_silu: null argument");
        if (M < 1 || N < 32 || N % 32 || K < 256 || K % 256)
            throw sd::Error("sd_op_gate_up_silu: need N a multiple of 32 and K of 256");
        OpWs& w = op_ws();
        std::lock_guard<std::mutex> lock(w.mu);
        const hipStream_t st = static_cast<hipStream_t>(stream);
        // the model's [gate | up] rows -> engine order, rows interleaved in groups of 16, tiled
        const size_t words = (size_t)N * K / 8, scales = (size_t)N * K / 32;
        grow(w.wpack, w.wpack_bytes, words * 4 + scales * 2);
        grow(w.wtmp, w.wtmp_bytes, words * 4 + scales * 2);
        auto* pw = static_cast<uint32_t*>(w.wpack);
        auto* ps = reinterpret_cast<sd::f16*>(pw + words);
        SD_HIP(hipMemcpyAsync(pw, Wq, words * 4, hipMemcpyDeviceToDevice, st));
        SD_HIP(hipMemcpyAsync(ps, Sc, scales * 2, hipMemcpyDeviceToDevice, st));
        sd::repack_w4(pw, words, st);
        sd::interleave_gate_up(pw, ps, N, K, w.wtmp, st);
        sd::tile_w4(pw, ps, N, K, w.wtmp, st);
        const auto* a = static_cast<const sd::f16*>(A);
        if (exact) {
            sd::gemv(a, pw, ps, nullptr, mid, 2, M, N, K, 4, 32, false, true, sd::gemv_plan(M, N, K, true, 2, 0), st);
            return;
        }
        const int c = cfg >= 0 ? cfg : sd::gemm_w4_plan(M, N, K, false, false, 0).cfg;
        if (!sd::gemm_w4_has_silu(c)) throw sd::Error("sd_op_gate_up_silu: configuration " + std::to_string(c) + " has no SiLU epilogue");
        sd::gemm_w4_silu(a, pw, ps, static_cast<sd::f16*>(mid), M, N, K, st, c, true);
    });
}

int sd_op_embed(const void* ids, int L, const void* Q, const void* S, const void* Bi, int d, int bits, int group, int asym,
                void* x, void* stream, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!ids || !Q || !S || !x || (asym && !Bi)) throw sd::Error("sd_op_embed: null argument");
        if (L < 1) throw sd::Error("sd_op_embed: need at least one id");
        sd::embed(static_cast<const uint32_t*>(ids), L, static_cast<const uint32_t*>(Q), static_cast<const sd::f16*>(S),
                  static_cast<const sd::f16*>(Bi), d, bits, group, asym != 0, static_cast<float*>(x),
                  static_cast<hipStream_t>(stream));
    });
}

int sd_op_add_norm(void* x, const void* y, const void* w, int d, const void* rows, int nrows, void* h16, void* h32,
                   void* stream, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!x || !w || (!h16 == !h32)) throw sd::Error("sd_op_add_norm: null argument (exactly one of h16, h32)");
        sd::YIn yi;
        yi.y16 = static_cast<const sd::f16*>(y);
        sd::add_norm(static_cast<float*>(x), yi, static_cast<const float*>(w), d, static_cast<const uint32_t*>(rows), nrows,
                     static_cast<sd::f16*>(h16), static_cast<float*>(h32), static_cast<hipStream_t>(stream));
    });
}

int sd_op_silu_mul(const void* big, int L, int I, void* mid, void* stream, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!big || !mid) throw sd::Error("sd_op_silu_mul: null argument");
        sd::silu_mul(static_cast<const sd::f16*>(big), nullptr, 0, L, I, false, static_cast<sd::f16*>(mid),
                     static_cast<hipStream_t>(stream));
    });
}

int sd_op_add_bias(void* y, int L, int N, const void* c, void* stream, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!y || !c) throw sd::Error("sd_op_add_bias: null argument");
        sd::add_bias(static_cast<sd::f16*>(y), L, N, static_cast<const float*>(c), static_cast<hipStream_t>(stream));
    });
}

int sd_op_conv(const void* big, int stride, int L, int C, const void* w, const void* hist, void* out, void* stream,
               char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!big || !w || !hist || !out) throw sd::Error("sd_op_conv: null argument");
        sd::conv_silu(static_cast<const sd::f16*>(big), stride, L, C, static_cast<const float*>(w),
                      static_cast<const sd::f16*>(hist), static_cast<float*>(out), sd::Segs{},
                      static_cast<hipStream_t>(stream));
    });
}

int sd_op_gnorm(const void* o, const void* big, int stride, int z_off, const void* w, int L, int H, int DV, void* out,
                void* stream, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!o || !big || !w || !out) throw sd::Error("sd_op_gnorm: null argument");
        const sd::GdnShape s{H, 128, DV, stride, 0, 0, z_off, 0};
        sd::gnorm(static_cast<const float*>(o), static_cast<const sd::f16*>(big), s, static_cast<const float*>(w), L,
                  static_cast<sd::f16*>(out), static_cast<hipStream_t>(stream));
    });
}

int sd_op_attention(const void* big, int stride, const void* qw, const void* kw, const void* rope, int L, int P, int HQ,
                    int HK, int HD, int RD, void* Q, void* Kc, void* Vt, int ctx, void* out, void* stream, char* err,
                    size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!big || !qw || !kw || !rope || !Q || !Kc || !Vt || !out) throw sd::Error("sd_op_attention: null argument");
        if (L < 1 || P < 0 || P + L > ctx) throw sd::Error("sd_op_attention: need 1 <= L and P + L <= ctx");
        if (ctx % 32) throw sd::Error("sd_op_attention: ctx must be a multiple of 32");
        if (HK < 1 || HQ % HK) throw sd::Error("sd_op_attention: q heads must be a multiple of kv heads");
        const sd::AttnShape as{HQ, HK, HD, RD, stride, ctx};
        // the engine's key split: query blocks of 16 that cannot fill the chip split the keys too
        const int nb = (L + 15) / 16;
        int ks = 1;
        if (L <= 256)
            while (ks < 8 && nb * HQ * ks < 256) ks *= 2;
        OpWs& w = op_ws();
        std::lock_guard<std::mutex> lock(w.mu);
        const hipStream_t st = static_cast<hipStream_t>(stream);
        grow(w.attn, w.attn_bytes, 256 + sd::attn_ws_floats(L, as) * 4);
        auto* lu = static_cast<uint32_t*>(w.attn);
        const uint32_t v[8] = {(uint32_t)L, (uint32_t)P, (uint32_t)ctx, P > 0 ? 1u : 0u, 0u, 0u, 0u, 0u};
        sd::set_u32x8(lu, v, st);
        sd::qk_prep(static_cast<const sd::f16*>(big), as, static_cast<const float*>(qw), static_cast<const float*>(kw),
                    static_cast<const float*>(rope), L, lu, sd::Segs{}, static_cast<sd::f16*>(Q), static_cast<sd::f16*>(Kc),
                    static_cast<sd::f16*>(Vt), st);
        // rotary_dim 64: the attention normalizes and rotates the queries itself, as in the engine (Q
        // is still written above for the caller)
        sd::attention_split(RD == 64 ? nullptr : static_cast<const sd::f16*>(Q), static_cast<const sd::f16*>(Kc),
                            static_cast<const sd::f16*>(Vt), static_cast<const sd::f16*>(big), as, L, lu, sd::Segs{}, ks,
                            reinterpret_cast<float*>(static_cast<uint8_t*>(w.attn) + 256), static_cast<sd::f16*>(out), st,
                            static_cast<const float*>(qw), static_cast<const float*>(rope));
    });
}

int sd_engine_trace(sd_engine* e, const uint32_t* ids, size_t n, const sd_snapshot* cache, const size_t* rows,
                    size_t n_rows, float* x_out, uint16_t* h_out, size_t cap, size_t* n_taps, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!e || !ids || (!rows && n_rows) || (cap && n_rows && (!x_out || !h_out)))
            throw sd::Error("sd_engine_trace: null argument");
        const size_t t = E(e)->trace(ids, n, S(cache), rows, n_rows, x_out, h_out, cap);
        if (n_taps) *n_taps = t;
    });
}

}  // extern "C"
