// The torso engine on one MI355X: weights resident in HBM, one dispatch plan per token length
// captured as a hipGraph, prefix snapshots as device-to-device copies.
// Reference: src/engine.rs (Engine::load 175-303, plan 396-524, forward 529-662, profile 668-711).
#include "engine.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace sd {

void launched(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw Error(std::string("launching ") + what + ": " + hipGetErrorString(e));
}

KernelEvents*& kernel_events() {
    thread_local KernelEvents* k = nullptr;
    return k;
}

namespace {

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

bool env_off(const char* name) {
    const char* v = std::getenv(name);
    return v && std::strcmp(v, "0") == 0;
}

// In-place fast Walsh-Hadamard transform, Sylvester order, unnormalized (src/engine.rs:714-727).
void fwht(float* x, size_t n) {
    for (size_t h = 1; h < n; h *= 2)
        for (size_t i = 0; i < n; i += 2 * h)
            for (size_t j = i; j < i + h; j++) {
                const float a = x[j], b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
}

}  // namespace

void decode_scale_codes(const uint8_t* src, size_t n, size_t g, uint16_t* dst, std::vector<double>& pw) {
    // pw: 2^(-i / 4096) in f64 for every exponent the rows use, grown on demand; the caller keeps it
    // for one load (the loader decodes one row at a time) and then drops it
    size_t jmax = 0;
    for (size_t r = 0; r < n; r++) jmax = std::max<size_t>(jmax, (size_t)src[4 * r + 2] | ((size_t)src[4 * r + 3] << 8));
    if (pw.size() < 127 * jmax + 1) {
        const size_t have = pw.size();
        pw.resize(127 * jmax + 1);
        for (size_t i = have; i < pw.size(); i++) pw[i] = std::pow(2.0, -(double)i / 4096.0);
    }
    const uint8_t* codes = src + 4 * n;
    for (size_t r = 0; r < n; r++) {
        const uint16_t mb = (uint16_t)(src[4 * r] | (src[4 * r + 1] << 8));
        const size_t j = (size_t)src[4 * r + 2] | ((size_t)src[4 * r + 3] << 8);
        const double m = (double)__builtin_bit_cast(f16, mb);
        uint16_t mag[128];
        bool have[128] = {};
        for (size_t i = 0; i < g; i++) {
            const uint8_t c = codes[r * g + i];
            const int k = c & 127;
            if (!have[k]) {
                mag[k] = __builtin_bit_cast(uint16_t, (f16)(float)(m * pw[k * j]));
                have[k] = true;
            }
            dst[r * g + i] = (uint16_t)(mag[k] | ((c & 128) << 8));
        }
    }
}

Engine::~Engine() {
    for (auto& kv : plans) kv.second.destroy();
    if (ev0) (void)hipEventDestroy(ev0);
    if (ev1) (void)hipEventDestroy(ev1);
    if (st) (void)hipStreamDestroy(st);
    for (void* p : device_allocs) (void)hipFree(p);
    if (pool.base) (void)hipFree(pool.base);
    for (void* p : host_allocs) (void)hipHostFree(p);
    if (head_dev) (void)hipFree(head_dev);
    if (hb.dev) (void)hipFree(hb.dev);
    if (hb.host) (void)hipHostFree(hb.host);
    for (auto& b : snap_pool) (void)hipFree(b.first);
}

void* Engine::snap_alloc(size_t bytes) {
    {
        std::lock_guard<std::mutex> lock(snap_mu);
        size_t best = snap_pool.size();
        for (size_t i = 0; i < snap_pool.size(); i++)
            if (snap_pool[i].second >= bytes && snap_pool[i].second <= 2 * bytes &&
                (best == snap_pool.size() || snap_pool[i].second < snap_pool[best].second))
                best = i;
        if (best < snap_pool.size()) {
            void* p = snap_pool[best].first;
            snap_pool.erase(snap_pool.begin() + best);
            return p;
        }
    }
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) throw Error(std::string("snapshot allocation: ") + hipGetErrorString(e));
    return p;
}

void Engine::snap_release(void* p, size_t bytes) const {
    std::lock_guard<std::mutex> lock(snap_mu);
    if (snap_pool.size() < 4) {
        snap_pool.emplace_back(p, bytes);
        return;
    }
    (void)hipFree(p);
}

void Plan::destroy() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    exec = nullptr;
    graph = nullptr;
}

void* Engine::dalloc(size_t bytes) {
    void* p = nullptr;
    SD_HIP(hipMalloc(&p, std::max<size_t>(bytes, 256)));
    device_allocs.push_back(p);
    return p;
}

void* Engine::halloc(size_t bytes) {
    void* p = nullptr;
    SD_HIP(hipHostMalloc(&p, std::max<size_t>(bytes, 256), hipHostMallocDefault));
    host_allocs.push_back(p);
    return p;
}

const TensorRef& Engine::tensor(const std::string& name) const {
    auto it = tensors.find(name);
    if (it == tensors.end()) throw Error("no tensor " + name);
    return it->second;
}

const void* Engine::dptr(const std::string& name) const {
    auto e = embed_parts.find(name);
    if (e != embed_parts.end()) return e->second;
    const TensorRef& t = tensor(name);
    for (const auto& s : shards)
        if (t.offset >= s.start && t.offset < s.start + s.bytes) {
            SD_CHECK(t.offset + t.bytes <= s.start + s.bytes, name + " crosses the end of its shard");
            return static_cast<const uint8_t*>(s.dev) + (t.offset - s.start);
        }
    throw Error(name + " is in no shard");
}

Mat Engine::mat(const std::string& name) const {
    const TensorRef& t = tensor(name + ".q");
    // the reference's formats (src/kernels.rs:550-576): int2/3/4, groups of a multiple of 32
    if (!(t.bits >= 2 && t.bits <= 4 && t.group >= 32 && t.group % 32 == 0 && t.K % t.group == 0))
        throw Error(name + ": unsupported weight format (" + std::to_string(t.bits) + " bits, group " +
                    std::to_string(t.group) + ", K " + std::to_string(t.K) + ")");
    Mat m;
    m.q = static_cast<const uint32_t*>(dptr(name + ".q"));
    m.s = static_cast<const f16*>(dptr(name + ".s"));
    if (t.asym) m.b = static_cast<const f16*>(dptr(name + ".b"));
    SD_CHECK(reinterpret_cast<uintptr_t>(m.q) % 16 == 0, name + ".q is not 16-byte aligned");
    m.N = (int)t.N;
    m.K = (int)t.K;
    m.bits = (int)t.bits;
    m.group = (int)t.group;
    m.asym = t.asym;
    SD_CHECK(tensor(name + ".s").bytes >= (uint64_t)m.N * (m.K / m.group) * 2, name + ".s: too few scales");
    // the tiled f16-dequant kernels need K a multiple of 128; the reference uses them for the
    // default format with N % 64 == 0 (src/engine.rs:434-442), the GEMV for everything else
    SD_CHECK(!m.deflt() || m.N % 64 != 0 || m.K % 128 == 0, name + ": K must be a multiple of 128");
    return m;
}

// The reference's GEMV (f32 dequant) serves M <= 20 rows, non-default formats and N % 64 != 0
// (src/engine.rs:419-442).  Every other matrix is in the engine layout (the load rewrites each
// default-format matrix of such a shape); the f16-dequant kernels read nothing else.
static bool gemv_rows(const Mat& m, bool short_rows) {
    const bool gemv = short_rows || !m.deflt() || m.N % 64 != 0;
    SD_CHECK(gemv || m.tiled, "a default-format matrix was not rewritten into the engine layout");
    return gemv;
}

const float* Engine::f32(const std::string& name, size_t count) const {
    const TensorRef& t = tensor(name);
    SD_CHECK(t.bytes >= count * 4, name + ": expected at least " + std::to_string(count) + " f32 values");
    const void* p = dptr(name);
    // the kernels read f32 vectors 16 bytes at a time; the model format places every tensor at a
    // multiple of 256 bytes (the reference binds each one as a storage-buffer slice,
    // src/engine.rs:325-357, whose offsets must be 256-aligned)
    SD_CHECK(reinterpret_cast<uintptr_t>(p) % 16 == 0, name + " is not 16-byte aligned");
    return static_cast<const float*>(p);
}

void Engine::load(const sd_config* c, const sd_tensor* ts, size_t nt, const char* const* shard_paths,
                  const uint64_t* shard_starts, const uint64_t* shard_bytes, size_t ns, const sd_embed* em) {
    SD_CHECK(c && ts && em, "sd_engine_load: null argument");
    cfg.d = (int)c->hidden_size;
    cfg.inter = (int)c->intermediate_size;
    cfg.hq = (int)c->num_attention_heads;
    cfg.hk = (int)c->num_key_value_heads;
    cfg.hd = (int)c->head_dim;
    cfg.rd = (int)c->rotary_dim;
    cfg.H = (int)c->linear_num_key_heads;
    cfg.dk = (int)c->linear_key_head_dim;
    cfg.dv = (int)c->linear_value_head_dim;
    cfg.theta = c->rope_theta;
    for (size_t i = 0; i < c->n_layers; i++) {
        const int k = c->layer_types[i];
        SD_CHECK(k == SD_LINEAR_ATTENTION || k == SD_FULL_ATTENTION || k == SD_ADAPTER,
                 "unsupported layer type " + std::to_string(k));
        kinds.push_back(k);
    }
    if (c->unrotate) unrotate.assign(c->unrotate, c->unrotate + cfg.d);
    {
        const int dd = cfg.d / 256;
        SD_CHECK(cfg.d % 256 == 0 && (dd <= 4 || dd == 6 || dd == 8 || dd == 10 || dd == 12 || dd == 16),
                 "hidden_size must be 256 x {1, 2, 3, 4, 6, 8, 10, 12, 16}");
    }

    for (size_t i = 0; i < nt; i++) {
        const sd_tensor& t = ts[i];
        SD_CHECK(t.name, "tensor without a name");
        if (t.had >= 0) throw Error(std::string(t.name) + ": online Hadamard rotation is not supported");
        tensors[t.name] = TensorRef{t.offset, t.bytes, t.N, t.K, t.bits, t.group, t.asym != 0};
    }

    int dev = 0;
    SD_HIP(hipGetDevice(&dev));
    hipDeviceProp_t prop;
    SD_HIP(hipGetDeviceProperties(&prop, dev));
    adapter = std::string(prop.name) + " (" + prop.gcnArchName + ", HIP)";
    SD_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    // timing only (the stream is synchronized before any result is read): no system-scope fence,
    // whose cache write-back and invalidation would be part of what the events time
    SD_HIP(hipEventCreateWithFlags(&ev0, hipEventDisableSystemFence));
    SD_HIP(hipEventCreateWithFlags(&ev1, hipEventDisableSystemFence));

    // Shards: one device buffer each, streamed from the file through a pinned staging buffer.
    const size_t chunk = size_t(64) << 20;
    uint8_t* stage = static_cast<uint8_t*>(halloc(chunk));
    for (size_t i = 0; i < ns; i++) {
        Shard s;
        s.start = shard_starts[i];
        s.bytes = shard_bytes[i];
        s.dev = dalloc(s.bytes);
        FILE* f = std::fopen(shard_paths[i], "rb");
        if (!f) throw Error(std::string(shard_paths[i]) + ": cannot open");
        for (uint64_t off = 0; off < s.bytes;) {
            const size_t n = (size_t)std::min<uint64_t>(chunk, s.bytes - off);
            if (std::fread(stage, 1, n, f) != n) {
                std::fclose(f);
                throw Error(std::string(shard_paths[i]) + ": shorter than the manifest says");
            }
            SD_HIP(hipMemcpy(static_cast<uint8_t*>(s.dev) + off, stage, n, hipMemcpyHostToDevice));
            off += n;
        }
        std::fclose(f);
        shards.push_back(s);
    }
    // Embedding parts: rows of [part0 | part1 | ...] split into one device array per part
    // (src/model.rs:260-283).
    {
        uint64_t gb = 0, wb = 0;  // bytes per row in GPU layout and as stored
        std::vector<bool> coded(em->n_parts, false);
        for (size_t p = 0; p < em->n_parts; p++) {
            coded[p] = em->u8 && std::strcmp(em->part_names[p], "embed.s") == 0;
            SD_CHECK(!coded[p] || em->part_bytes[p] % 2 == 0, "embed: the scale part must hold f16 values");
            gb += em->part_bytes[p];
            wb += coded[p] ? 4 + em->part_bytes[p] / 2 : em->part_bytes[p];
        }
        SD_CHECK(gb == em->row_bytes, "embed: part sizes do not add up to row_bytes");
        const uint64_t rb = em->wire_row_bytes ? em->wire_row_bytes : em->row_bytes;
        SD_CHECK(wb == rb, "embed: the stored parts do not add up to the stored row size");
        FILE* f = std::fopen(em->rows_path, "rb");
        if (!f) throw Error(std::string(em->rows_path) + ": cannot open");
        std::fseek(f, 0, SEEK_END);
        const long size = std::ftell(f);
        std::fseek(f, 0, SEEK_SET);
        if ((uint64_t)size != em->vocab * rb) {
            std::fclose(f);
            throw Error(std::string(em->rows_path) + ": " + std::to_string(size) + " bytes, expected " +
                        std::to_string(em->vocab) + " rows of " + std::to_string(rb));
        }
        std::vector<std::vector<uint8_t>> parts(em->n_parts);
        for (size_t p = 0; p < em->n_parts; p++) parts[p].resize(em->vocab * em->part_bytes[p]);
        const size_t rows_per = std::max<size_t>(1, chunk / rb);
        std::vector<uint8_t> buf(rows_per * rb);
        std::vector<double> pw;  // the scale-code power table, for this load only
        for (uint64_t r0 = 0; r0 < em->vocab; r0 += rows_per) {
            const size_t nr = (size_t)std::min<uint64_t>(rows_per, em->vocab - r0);
            if (std::fread(buf.data(), rb, nr, f) != nr) {
                std::fclose(f);
                throw Error(std::string(em->rows_path) + ": read failed");
            }
            for (size_t r = 0; r < nr; r++) {
                size_t off = 0;
                for (size_t p = 0; p < em->n_parts; p++) {
                    uint8_t* dst = parts[p].data() + (r0 + r) * em->part_bytes[p];
                    const uint8_t* src = buf.data() + r * rb + off;
                    if (coded[p]) {
                        const size_t g = em->part_bytes[p] / 2;
                        decode_scale_codes(src, 1, g, reinterpret_cast<uint16_t*>(dst), pw);
                        off += 4 + g;
                    } else {
                        std::memcpy(dst, src, em->part_bytes[p]);
                        off += em->part_bytes[p];
                    }
                }
            }
        }
        std::fclose(f);
        for (size_t p = 0; p < em->n_parts; p++) {
            void* dptr_ = dalloc(parts[p].size());
            SD_HIP(hipMemcpy(dptr_, parts[p].data(), parts[p].size(), hipMemcpyHostToDevice));
            embed_parts[em->part_names[p]] = dptr_;
        }
        vocab = (int)em->vocab;
    }
    {
        const TensorRef& t = tensor("embed.q");
        emb.bits = (int)t.bits;
        emb.group = (int)t.group;
        emb.asym = t.asym;
        emb.q = static_cast<const uint32_t*>(dptr("embed.q"));
        emb.s = static_cast<const f16*>(dptr("embed.s"));
        emb.b = emb.asym ? static_cast<const f16*>(dptr("embed.b")) : nullptr;
    }

    // Per-layer weights and live state.  GDN state and conv history of every linear layer live in
    // one arena ([all states | all histories]) so that a snapshot is a single copy.
    const int C = 2 * cfg.H * cfg.dk + cfg.H * cfg.dv;
    const size_t state_bytes = (size_t)cfg.H * cfg.dk * cfg.dv * 4, hist_bytes = align256((size_t)3 * C * 2);
    n_linear = 0;
    for (int k : kinds) n_linear += k == SD_LINEAR_ATTENTION;
    arena_state_bytes = n_linear * state_bytes;
    arena_bytes = arena_state_bytes + n_linear * hist_bytes;
    arena = static_cast<uint8_t*>(dalloc(arena_bytes));
    SD_HIP(hipMemset(arena, 0, arena_bytes));
    const size_t kv_bytes = (size_t)cfg.hk * SD_CONTEXT * cfg.hd * 2;
    int li = 0;
    for (size_t i = 0; i < kinds.size(); i++) {
        const std::string p = "layers." + std::to_string(i) + ".";
        LayerW L;
        L.kind = kinds[i];
        L.in_norm = f32(p + "in_norm", cfg.d);
        if (L.kind == SD_ADAPTER) {
            L.proj = mat(p + "proj");
            L.bias = f32(p + "bias", cfg.d);
            layers.push_back(L);
            continue;
        }
        if (L.kind == SD_LINEAR_ATTENTION) {
            SD_CHECK(cfg.dk == 128 && cfg.dv == 128, "gated delta net: only 128-wide key/value heads are supported");
            L.in_proj = mat(p + "in_proj");
            SD_CHECK(L.in_proj.N >= C + 2 * cfg.H * 1 + cfg.H * cfg.dv, p + "in_proj: too few rows for q|k|v|z|a|b");
            L.conv = f32(p + "conv", (size_t)C * 4);
            L.negA = f32(p + "neg_exp_A", cfg.H);
            L.dtb = f32(p + "dt_bias", cfg.H);
            L.gnorm = f32(p + "gnorm", cfg.dv);
            L.out_proj = mat(p + "out_proj");
            L.state_off = li * state_bytes;
            L.hist_off = arena_state_bytes + li * hist_bytes;
            L.state = reinterpret_cast<float*>(arena + L.state_off);
            L.hist = reinterpret_cast<f16*>(arena + L.hist_off);
            li++;
        } else {
            SD_CHECK(cfg.hd == 256, "attention: only head_dim 256 is supported");
            // rotate-half pairs dims d and d + rotary_dim / 2 (the reference's RD2 = rd / 2)
            SD_CHECK(cfg.rd >= 2 && cfg.rd % 2 == 0 && cfg.rd <= cfg.hd,
                     "attention: rotary_dim must be even, from 2 to head_dim");
            SD_CHECK(cfg.hk > 0 && cfg.hq % cfg.hk == 0, "attention: q heads must be a multiple of kv heads");
            L.qkv = mat(p + "qkv");
            SD_CHECK(L.qkv.N >= 2 * cfg.hq * cfg.hd + 2 * cfg.hk * cfg.hd, p + "qkv: too few rows");
            L.q_norm = f32(p + "q_norm", cfg.hd);
            L.k_norm = f32(p + "k_norm", cfg.hd);
            L.o_proj = mat(p + "o_proj");
            L.kc = static_cast<f16*>(dalloc(kv_bytes));
            L.vc = static_cast<f16*>(dalloc(kv_bytes));
            SD_HIP(hipMemset(L.kc, 0, kv_bytes));
            SD_HIP(hipMemset(L.vc, 0, kv_bytes));
            attn_layers.push_back((int)i);
        }
        L.post_norm = f32(p + "post_norm", cfg.d);
        L.gate_up = mat(p + "gate_up");
        L.down = mat(p + "down");
        SD_CHECK(L.gate_up.N == 2 * cfg.inter && L.down.K == cfg.inter, p + "gate_up/down: shapes do not match intermediate_size");
        layers.push_back(L);
    }
    final_norm = f32("final_norm", cfg.d);
    // Matmul weights into the engine nibble order, gate_up rows interleaved, then the tiled layout,
    // each matrix once (matrices are told apart by their memory).
    {
        std::vector<Mat*> all;
        for (LayerW& L : layers)
            for (Mat* m : {&L.in_proj, &L.out_proj, &L.qkv, &L.o_proj, &L.gate_up, &L.down, &L.proj})
                if (m->q) all.push_back(m);
        // Matrices that share memory must agree in shape and format: the rewrite into the engine
        // layout below is done once per memory, and a GEMM reading the rewritten words as another
        // shape would read the model's bit order as the engine's.
        for (const Mat* a : all)
            for (const Mat* b : all)
                if (a->q == b->q && (a->N != b->N || a->K != b->K || a->bits != b->bits || a->group != b->group ||
                                     a->asym != b->asym))
                    throw Error("two matrices share memory with different shapes or formats (" + std::to_string(a->N) +
                                " x " + std::to_string(a->K) + " and " + std::to_string(b->N) + " x " +
                                std::to_string(b->K) + ")");
        // Only int4 g32 symmetric matrices of a tileable shape are rewritten (the kernels with f16
        // dequant read nothing else); every other matrix keeps the reference's layout and bit order,
        // which the GEMV reads.
        auto rewritable = [&](const Mat* m) { return m->deflt() && w4_tileable(m->N, m->K); };
        std::vector<const uint32_t*> done;
        size_t tmp_bytes = 0;
        for (const Mat* m : all) {
            if (!rewritable(m)) continue;
            tmp_bytes = std::max(tmp_bytes, (size_t)m->N * m->K / 2 + (size_t)m->N * m->K / 16);
            if (std::find(done.begin(), done.end(), m->q) != done.end()) continue;
            done.push_back(m->q);
            repack_w4(const_cast<uint32_t*>(m->q), (size_t)m->N * m->K / 8, st);
        }
        // gate_up rows interleaved in groups of 16, so the GEMM's epilogue can apply silu * mul
        // (possible when no other matrix shares a gate_up's memory)
        std::vector<const Mat*> gus;
        for (const LayerW& L : layers)
            if (L.kind != SD_ADAPTER && L.gate_up.q) gus.push_back(&L.gate_up);
        gu_il = !gus.empty() && cfg.inter % 16 == 0;
        for (const Mat* g : gus)
            if (!rewritable(g)) gu_il = false;
        for (const Mat* g : gus)
            for (const Mat* m : all)
                if (m->q == g->q && m != g && std::find(gus.begin(), gus.end(), m) == gus.end()) gu_il = false;
        void* tmp = nullptr;  // load-time scratch, freed below
        SD_HIP(hipMalloc(&tmp, std::max<size_t>(tmp_bytes, 256)));
        try {
            std::vector<const uint32_t*> il_done;
            for (const Mat* g : gus) {
                if (!gu_il || std::find(il_done.begin(), il_done.end(), g->q) != il_done.end()) continue;
                il_done.push_back(g->q);
                interleave_gate_up(const_cast<uint32_t*>(g->q), const_cast<f16*>(g->s), g->N, g->K, tmp, st);
            }
            // the tiled layout for every matrix that has one (each matrix sharing memory with a
            // tiled one is tiled with it)
            std::vector<const uint32_t*> tiled_done;
            for (Mat* m : all) {
                m->tiled = rewritable(m);
                if (!m->tiled || std::find(tiled_done.begin(), tiled_done.end(), m->q) != tiled_done.end()) continue;
                tiled_done.push_back(m->q);
                tile_w4(const_cast<uint32_t*>(m->q), const_cast<f16*>(m->s), m->N, m->K, tmp, st);
            }
            SD_HIP(hipStreamSynchronize(st));
        } catch (...) {
            (void)hipStreamSynchronize(st);
            (void)hipFree(tmp);
            throw;
        }
        SD_HIP(hipFree(tmp));
    }

    // RoPE table, angles in f64 (src/engine.rs:259-267).
    {
        std::vector<float> table((size_t)SD_CONTEXT * std::max(cfg.rd, 2));
        for (int t = 0; t < SD_CONTEXT; t++)
            for (int i = 0; i < cfg.rd / 2; i++) {
                const double a = (double)t / std::pow(cfg.theta, (double)(2 * i) / (double)cfg.rd);
                table[(size_t)t * cfg.rd + 2 * i] = (float)std::cos(a);
                table[(size_t)t * cfg.rd + 2 * i + 1] = (float)std::sin(a);
            }
        rope = static_cast<float*>(dalloc(table.size() * 4));
        SD_HIP(hipMemcpy(rope, table.data(), table.size() * 4, hipMemcpyHostToDevice));
    }
    use_graphs = !env_off("SD_GRAPHS");
    {
        const char* c = std::getenv("STRANDS_DECIDER_CHECKED");
        checked = c && std::strcmp(c, "1") == 0;
        if (checked) use_graphs = false;  // every step runs eagerly
    }
    for (const LayerW& L : layers) {
        if (L.kind == SD_LINEAR_ATTENTION) max_n = std::max(max_n, L.in_proj.N);
        if (L.kind == SD_FULL_ATTENTION) max_n = std::max(max_n, L.qkv.N);
        if (L.kind != SD_ADAPTER) max_n = std::max(max_n, L.gate_up.N);
    }
    max_n = std::max(max_n, cfg.d);
}

void Engine::ensure_pool(int l) {
    const int cap = l <= 128 ? 128 : (int)std::min<size_t>(SD_CONTEXT, size_t(1) << (32 - __builtin_clz((unsigned)l - 1)));
    if (pool.cap >= cap) return;
    // A bigger pool serves every shorter length too; plans bound to the old one are rebuilt.
    for (auto& kv : plans) kv.second.destroy();
    plans.clear();
    if (pool.base) SD_HIP(hipFree(pool.base));
    pool = Pool{};
    const int C = 2 * cfg.H * cfg.dk + cfg.H * cfg.dv;
    const int orow = std::max({cfg.H * cfg.dv, cfg.hq * cfg.hd, cfg.d});
    GdnShape gs{cfg.H, cfg.dk, cfg.dv, 0, 0, 0, 0, C};
    AttnShape as{cfg.hq, cfg.hk, cfg.hd, cfg.rd, 0, SD_CONTEXT};
    const size_t ypart = (size_t)8 * cap * cfg.d;
    // gate_up partials: 8 slots for short inputs, fewer for long ones (whose grids need no split)
    const size_t gpart = (size_t)(cap <= 256 ? 8 : 1) * cap * 2 * cfg.inter;
    // the upload block: lu, ids, rows, Segs row / chunk / sequence tables
    Pool up;
    up.off_ids = 256;
    up.off_rows = up.off_ids + align256((size_t)cap * 4);
    up.off_seg_row = up.off_rows + align256((size_t)cap * 4);
    up.off_seg_chunk = up.off_seg_row + align256((size_t)cap * 4);
    up.off_seg_seq = up.off_seg_chunk + align256((size_t)(cap / 64 + SD_MAX_SEQS) * 4);
    up.up_bytes = up.off_seg_seq + align256((size_t)SD_MAX_SEQS * 8);
    const size_t sizes[] = {
        up.up_bytes,                                   // upload block
        (size_t)cap * cfg.d * 4,                       // x
        (size_t)cap * cfg.d * 2,                       // h
        (size_t)cap * max_n * 2,                       // big
        (size_t)cap * cfg.inter * 2,                   // mid
        (size_t)cap * C * 4,                           // qkvc
        (size_t)cap * cfg.H * cfg.dv * 4,              // of
        (size_t)cap * orow * 2,                        // o
        (size_t)cap * cfg.d * 2,                       // y
        (size_t)cfg.hq * cap * cfg.hd * 2,             // q
        (size_t)cap * cfg.d * 4,                       // out
        gdn_ws_bytes(cap, gs),                         // GDN chunk workspace
        attn_ws_floats(std::min(cap, 256), as) * 4,    // attention key-split workspace
        ypart * 4,                                     // split-K partials of y
        gpart * 4,                                     // split-K partials of gate_up
        (size_t)cap * cfg.d * 4,                       // xc: a compact last layer's residual rows
        (size_t)cap * orow * 2,                        // oc: a compact last layer's mixer output rows
    };
    size_t total = 0;
    for (size_t s : sizes) total += align256(s);
    void* base = nullptr;
    SD_HIP(hipMalloc(&base, total));
    pool.base = base;
    pool.cap = cap;
    uint8_t* p = static_cast<uint8_t*>(base);
    void* ptrs[sizeof(sizes) / sizeof(sizes[0])];
    for (size_t i = 0; i < sizeof(sizes) / sizeof(sizes[0]); i++) {
        ptrs[i] = p;
        p += align256(sizes[i]);
    }
    uint8_t* upb = static_cast<uint8_t*>(ptrs[0]);
    pool.up_bytes = up.up_bytes;
    pool.off_ids = up.off_ids;
    pool.off_rows = up.off_rows;
    pool.off_seg_row = up.off_seg_row;
    pool.off_seg_chunk = up.off_seg_chunk;
    pool.off_seg_seq = up.off_seg_seq;
    lu = reinterpret_cast<uint32_t*>(upb);
    pool.ids = reinterpret_cast<uint32_t*>(upb + up.off_ids);
    pool.rows = reinterpret_cast<uint32_t*>(upb + up.off_rows);
    pool.seg_row = reinterpret_cast<uint32_t*>(upb + up.off_seg_row);
    pool.seg_chunk = reinterpret_cast<uint32_t*>(upb + up.off_seg_chunk);
    pool.seg_seq = reinterpret_cast<uint32_t*>(upb + up.off_seg_seq);
    pool.seg_chunk_cap = cap / 64 + SD_MAX_SEQS;
    pool.x = (float*)ptrs[1];
    pool.h = (f16*)ptrs[2];
    pool.big = (f16*)ptrs[3];
    pool.mid = (f16*)ptrs[4];
    pool.qkvc = (float*)ptrs[5];
    pool.of = (float*)ptrs[6];
    pool.o = (f16*)ptrs[7];
    pool.y = (f16*)ptrs[8];
    pool.q = (f16*)ptrs[9];
    pool.out = (float*)ptrs[10];
    gdn_ws_carve(ptrs[11], cap, gs, pool.gdn);
    pool.attn_ws = (float*)ptrs[12];
    pool.attn_rows = std::min(cap, 256);
    pool.ypart = (float*)ptrs[13];
    pool.ypart_elems = ypart;
    pool.gpart = (float*)ptrs[14];
    pool.gpart_elems = gpart;
    pool.xc = (float*)ptrs[15];
    pool.oc = (f16*)ptrs[16];
    SD_HIP(hipMemset(pool.x, 0, (size_t)cap * cfg.d * 4));
    SD_HIP(hipMemset(upb, 0, up.up_bytes));
    if (up_h_bytes < up.up_bytes) {
        up_h = static_cast<uint8_t*>(halloc(up.up_bytes));
        up_h_bytes = up.up_bytes;
    }
    up_dirty = 0;
    if (out_h_cap < cap) {
        out_h = static_cast<float*>(halloc((size_t)cap * cfg.d * 4));
        out_h_cap = cap;
    }
}

void Engine::mm(std::vector<Step>& steps, const char* label, const f16* A, const Mat& m, f16* Y, int L,
                bool short_rows) {
    if (gemv_rows(m, short_rows)) {
        const GemvPlan gp = gemv_plan(L, m.N, m.K, m.tiled, 0, 0);
        steps.push_back({label, [=](hipStream_t s) {
            gemv(A, m.q, m.s, m.b, Y, 0, L, m.N, m.K, m.bits, m.group, m.asym, m.tiled, gp, s);
        }});
        return;
    }
    const int cfg_ = gemm_w4_plan(L, m.N, m.K, false, false, 0).cfg;
    steps.push_back({label, [=](hipStream_t s) { gemm_w4(A, m.q, m.s, Y, nullptr, L, m.N, m.K, false, 1, s, cfg_, m.tiled); }});
}

YIn Engine::mm_y(std::vector<Step>& steps, const char* label, const f16* A, const Mat& m, int L, bool short_rows) {
    // A projection whose output only feeds the residual add: split K until the grid covers the
    // chip, the add + RMSNorm sums the partials.
    if (gemv_rows(m, short_rows)) {
        const GemvPlan gp = gemv_plan(L, m.N, m.K, m.tiled, 1, pool.ypart_elems);
        float* part = pool.ypart;
        steps.push_back({label, [=](hipStream_t s) {
            gemv(A, m.q, m.s, m.b, part, 1, L, m.N, m.K, m.bits, m.group, m.asym, m.tiled, gp, s);
        }});
        YIn y;
        y.yp = part;
        y.ks = gp.ks;
        y.slot = (size_t)L * m.N;
        return y;
    }
    const bool exact = false;
    const GemmPlan gp = gemm_w4_plan(L, m.N, m.K, exact, true, pool.ypart_elems);
    const int cfg_ = gp.cfg, ks = gp.ks;
    float* part = pool.ypart;
    steps.push_back({label, [=](hipStream_t s) {
        gemm_w4(A, m.q, m.s, nullptr, part, L, m.N, m.K, exact, ks, s, cfg_, m.tiled);
    }});
    YIn y;
    y.yp = part;
    y.ks = ks;
    y.slot = (size_t)L * m.N;
    return y;
}

Plan& Engine::plan(int L, int nseq, bool short_seqs, int tree, bool cache_only, int rows_read) {
    // A forward that reads at most half its rows runs its last layer's tail (after the token mixer:
    // o_proj or out_proj, the residual add + norm, the MLP) on the read rows only, gathered into a
    // compact block; the final norm then reads them there.  The mixer itself runs on every row (its
    // output rows depend on all earlier rows).  An adapter as the last layer keeps the full tail.
    const int compact = !cache_only && rows_read > 0 && 2 * rows_read <= L && !layers.empty() &&
                                layers.back().kind != SD_ADAPTER
                            ? rows_read
                            : 0;
    const uint64_t key = (uint64_t)(cache_only ? 1u : 0u) << 63 | (uint64_t)compact << 46 | (uint64_t)tree << 32 |
                         (uint64_t)L << 8 | (uint64_t)nseq << 1 | (short_seqs ? 1u : 0u);
    auto it = plans.find(key);
    if (it != plans.end()) {
        it->second.used = ++plan_clock;
        return it->second;
    }
    // Every forward ends with the device idle, so no evicted graph is still running.
    if (plans.size() >= kMaxPlans) {
        auto lru = std::min_element(plans.begin(), plans.end(),
                                    [](const auto& a, const auto& b) { return a.second.used < b.second.used; });
        lru->second.destroy();
        plans.erase(lru);
    }
    Plan pl;
    pl.L = L;
    const bool sr = nseq ? short_seqs : L <= 20;  // the reference's GEMV rows
    Segs sg;
    if (nseq) sg = Segs{pool.seg_row, pool.seg_chunk, pool.seg_seq};
    const int nch = (L + 63) / 64 + (nseq ? nseq - 1 : 0);  // most chunks L rows can split into
    // Short inputs (at most 64 tokens per sequence on average: a question, a batch of them) run the
    // delta rule token by token; longer ones in chunks of 64 (prep + scan).
    const bool recur = L <= 64 * std::max(nseq, 1);
    auto& steps = pl.steps;
    const Pool P = pool;
    const int d = cfg.d, I = cfg.inter;
    const int C = 2 * cfg.H * cfg.dk + cfg.H * cfg.dv;
    const EmbedW E = emb;
    const uint32_t* luv = lu;
    steps.push_back({"embed", [=](hipStream_t s) { embed(P.ids, L, E.q, E.s, E.b, d, E.bits, E.group, E.asym, P.x, s); }});
    YIn y;  // the sublayer output the next add + norm consumes (none before layer 0)
    for (size_t i = 0; i < layers.size(); i++) {
        const LayerW W = layers[i];
        // cache_only (a forward that reads no hidden row, such as a state encoded for its snapshot):
        // the last layer's output feeds nothing, so it runs only the steps that write the cache (the
        // K/V rows, or the recurrent state and conv history); an adapter writes none
        const bool cache_end = cache_only && i + 1 == layers.size();
        if (cache_end && W.kind == SD_ADAPTER) break;
        // this layer's tail runs on the R compact rows (the last layer of a compact plan), else on all L
        const bool tail_c = compact > 0 && i + 1 == layers.size();
        const int R = tail_c ? compact : L;
        float* const xt = tail_c ? P.xc : P.x;
        {
            const YIn yin = y;
            steps.push_back({"norm", [=](hipStream_t s) { add_norm(P.x, yin, W.in_norm, d, nullptr, L, P.h, nullptr, s); }});
        }
        if (W.kind == SD_ADAPTER) {
            mm(steps, "proj", P.h, W.proj, P.y, L, sr);
            steps.push_back({"bias", [=](hipStream_t s) { add_bias(P.y, L, d, W.bias, s); }});
            y = YIn{};
            y.y16 = P.y;
            continue;
        }
        if (W.kind == SD_LINEAR_ATTENTION) {
            const int n = W.in_proj.N;
            const GdnShape gs{cfg.H, cfg.dk, cfg.dv, n, C + cfg.H * cfg.dv, C + cfg.H * cfg.dv + cfg.H, C, C};
            mm(steps, "in_proj", P.h, W.in_proj, P.big, L, sr);
            // conv and the delta rule read the prefix's history and state in place (from the snapshot
            // the lu block names, else the live arena) and write the live arena
            f16* hist_upd = nseq ? nullptr : W.hist;  // several sequences leave no history
            if (tree) {
                // The state (rows 0 .. tree - 1) in chunks, as its own forward without a prefix: a
                // fresh state, the cleared history, its final state and history into the live arena.
                // The branches in chunks too, each from that state: their chunks' prep runs in the
                // state's prep launch (a branch's rows before its first are the state's last ones),
                // then, after the state's scan, a scan of the branches as sequences starting from the
                // live state (lu has has_cache set and names no snapshot), through the sequence
                // tables shifted past the state; it keeps no state.
                const int S = tree, nbr = nseq - 1;
                const ConvIn cin{W.conv, W.hist, sg.row, W.hist_off};
                steps.push_back({"gdn", [=](hipStream_t s) {
                    gdn_prep(nullptr, P.big, gs, W.negA, W.dtb, L, P.gdn, cin, sg, nch, luv, s);
                }});
                steps.push_back({"gdn", [=](hipStream_t s) {
                    gdn_scan(gs, S, P.gdn, W.state, nullptr, 0, P.of, Segs{}, 0, s, W.state_off, W.hist, P.big, W.hist_off);
                }});
                const Segs sgb{sg.row, sg.chunk, sg.seq + 1};
                steps.push_back({"gdn", [=](hipStream_t s) {
                    gdn_scan(gs, L, P.gdn, W.state, luv, 0, P.of, sgb, nbr, s, W.state_off, nullptr, P.big, W.hist_off);
                }});
            } else if (recur && nseq) {
                // several sequences update no history: the recurrence computes the conv itself
                const ConvIn cin{W.conv, W.hist, sg.row, W.hist_off};
                steps.push_back({"gdn", [=](hipStream_t s) {
                    gdn_recur(nullptr, P.big, gs, W.negA, W.dtb, L, W.state, luv, 0, P.of, nullptr, sg, nseq, s,
                              W.state_off, W.hist_off, cin);
                }});
            } else if (recur) {
                // one sequence: the conv reads the old history before the recurrence updates it
                steps.push_back({"conv", [=](hipStream_t s) {
                    conv_silu(P.big, n, L, C, W.conv, W.hist, P.qkvc, sg, s, luv, W.hist_off);
                }});
                steps.push_back({"gdn", [=](hipStream_t s) {
                    gdn_recur(P.qkvc, P.big, gs, W.negA, W.dtb, L, W.state, luv, 0, P.of, hist_upd, sg, nseq, s, W.state_off,
                              W.hist_off);
                }});
            } else {
                // the chunked path computes the conv inside prep (no conv output in HBM); the history
                // is updated by the scan, after every prep workgroup has read the old one
                const ConvIn cin{W.conv, W.hist, sg.row, W.hist_off};
                steps.push_back({"gdn", [=](hipStream_t s) {
                    gdn_prep(nullptr, P.big, gs, W.negA, W.dtb, L, P.gdn, cin, sg, nch, luv, s);
                }});
                steps.push_back({"gdn", [=](hipStream_t s) {
                    gdn_scan(gs, L, P.gdn, W.state, luv, 0, P.of, sg, nseq, s, W.state_off, hist_upd, P.big, W.hist_off);
                }});
            }
            if (cache_end) break;
            steps.push_back({"gnorm", [=](hipStream_t s) { gnorm(P.of, P.big, gs, W.gnorm, L, P.o, s); }});
            if (tail_c) {
                const size_t ob = (size_t)W.out_proj.K * 2, xb = (size_t)d * 4;
                steps.push_back({"gather", [=](hipStream_t s) { gather_rows2(P.o, P.oc, ob, P.x, P.xc, xb, P.rows, R, s); }});
            }
            y = mm_y(steps, "out_proj", tail_c ? P.oc : P.o, W.out_proj, R, sr);
        } else {
            const AttnShape as{cfg.hq, cfg.hk, cfg.hd, cfg.rd, W.qkv.N, SD_CONTEXT};
            const float* rp = rope;
            if (cache_end && W.qkv.tiled && W.qkv.N == 2 * cfg.hq * cfg.hd + 2 * cfg.hk * cfg.hd && !gemv_rows(W.qkv, sr)) {
                // Only the cache rows are needed: K and V, the last 2 hk hd output columns (in the
                // tiled layout a column range starts n0 K / 32 blocks in), then qk_prep over a view
                // with no q heads.  The GEMM runs the full qkv GEMM's configuration, whose sums per
                // output element do not depend on N: the cache rows are those a forward reading rows
                // writes, bit for bit.
                const int n0 = 2 * cfg.hq * cfg.hd;
                Mat kv = W.qkv;
                kv.q += (size_t)n0 * kv.K / 8;
                kv.s += (size_t)n0 * (kv.K / 32);
                kv.N -= n0;
                const int cf = gemm_w4_plan(L, W.qkv.N, W.qkv.K, false, false, 0).cfg;
                steps.push_back({"qkv", [=](hipStream_t s) {
                    gemm_w4(P.h, kv.q, kv.s, P.big, nullptr, L, kv.N, kv.K, false, 1, s, cf, true);
                }});
                const AttnShape akv{0, cfg.hk, cfg.hd, cfg.rd, kv.N, SD_CONTEXT};
                steps.push_back({"qk_prep", [=](hipStream_t s) {
                    qk_prep(P.big, akv, W.q_norm, W.k_norm, rp, L, luv, sg, nullptr, W.kc, W.vc, s);
                }});
                break;
            }
            mm(steps, "qkv", P.h, W.qkv, P.big, L, sr);
            // rotary_dim 64: each attention workgroup normalizes and rotates its own queries, and
            // qk_prep writes only the K and V cache rows (which other workgroups read)
            f16* const qbuf = cfg.rd == 64 ? nullptr : P.q;
            steps.push_back({"qk_prep", [=](hipStream_t s) {
                qk_prep(P.big, as, W.q_norm, W.k_norm, rp, L, luv, sg, qbuf, W.kc, W.vc, s);
            }});
            if (cache_end) break;
            const int nb = (L + 15) / 16;
            int ks = 1;
            if (L <= P.attn_rows)
                while (ks < 8 && nb * cfg.hq * ks < 256) ks *= 2;
            steps.push_back({"attn", [=](hipStream_t s) {
                attention_split(qbuf, W.kc, W.vc, P.big, as, L, luv, sg, ks, P.attn_ws, P.o, s, W.q_norm, rp);
            }});
            if (tail_c) {
                const size_t ob = (size_t)W.o_proj.K * 2, xb = (size_t)d * 4;
                steps.push_back({"gather", [=](hipStream_t s) { gather_rows2(P.o, P.oc, ob, P.x, P.xc, xb, P.rows, R, s); }});
            }
            y = mm_y(steps, "o_proj", tail_c ? P.oc : P.o, W.o_proj, R, sr);
        }
        {
            const YIn yin = y;
            steps.push_back({"norm", [=](hipStream_t s) { add_norm(xt, yin, W.post_norm, d, nullptr, R, P.h, nullptr, s); }});
        }
        {
            // gate_up only feeds silu * mul: from 65 to 2560 rows it runs unsplit with silu * mul in
            // the GEMM's epilogue (measured on MI355X at 120 rows: 15.7 us against 13.7 us split in
            // two plus 4.9 us of silu_mul; the measured plans up to 2560 rows are of the epilogue
            // kernels); otherwise silu_mul sums the split-K partials itself.  The
            // GEMV rows apply silu * mul in the GEMV's epilogue when the weights are interleaved.
            const Mat m = W.gate_up;
            const bool exact = gemv_rows(m, sr);
            const bool il = gu_il;
            const int cfu = !exact && m.K % 256 == 0 && R > 64 && R <= 2560 ? gemm_w4_plan(R, m.N, m.K, false, false, 0).cfg : -1;
            if (exact) {
                const bool fused = il && m.tiled;
                const GemvPlan gp = gemv_plan(R, m.N, m.K, m.tiled, fused ? 2 : 0, 0);
                steps.push_back({"gate_up", [=](hipStream_t s) {
                    gemv(P.h, m.q, m.s, m.b, fused ? (void*)P.mid : (void*)P.big, fused ? 2 : 0, R, m.N, m.K, m.bits, m.group,
                         m.asym, m.tiled, gp, s);
                }});
                if (!fused) steps.push_back({"silu", [=](hipStream_t s) { silu_mul(P.big, nullptr, 0, R, I, il, P.mid, s); }});
            } else if (il && gemm_w4_has_silu(cfu)) {
                const int cg = cfu;
                steps.push_back({"gate_up", [=](hipStream_t s) {
                    gemm_w4_silu(P.h, m.q, m.s, P.mid, R, m.N, m.K, s, cg, m.tiled);
                }});
            } else {
                const GemmPlan plan_ = gemm_w4_plan(R, m.N, m.K, exact, true, P.gpart_elems);
                const int cg = plan_.cfg, ks = plan_.ks;
                float* gp = ks > 1 ? P.gpart : nullptr;  // unsplit: f16 straight into big
                steps.push_back({"gate_up", [=](hipStream_t s) {
                    gemm_w4(P.h, m.q, m.s, P.big, gp, R, m.N, m.K, exact, ks, s, cg, m.tiled);
                }});
                steps.push_back({"silu", [=](hipStream_t s) { silu_mul(P.big, gp, ks, R, I, il, P.mid, s); }});
            }
        }
        y = mm_y(steps, "down", P.mid, W.down, R, sr);
    }
    pl.last_y = y;  // (unused by a cache_only plan: no hidden row is read)
    pl.compact = compact;
    if (use_graphs) {
        SD_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        try {
            for (auto& s : steps) s.run(st);
        } catch (...) {
            hipGraph_t g = nullptr;
            (void)hipStreamEndCapture(st, &g);
            if (g) (void)hipGraphDestroy(g);
            throw;
        }
        SD_HIP(hipStreamEndCapture(st, &pl.graph));
        SD_HIP(hipGraphInstantiate(&pl.exec, pl.graph, nullptr, nullptr, 0));
    }
    pl.used = ++plan_clock;
    return plans.emplace(key, std::move(pl)).first->second;
}

void Engine::upload(const uint32_t* ids, size_t n, const size_t* rows, size_t n_rows, size_t P, bool has_cache,
                    uint32_t chunks, uint32_t nseq, const Snapshot* cache, uint32_t tree) {
    // lu, ids and rows (and the Segs tables a batch wrote before) in one host-to-device copy; the lu
    // block names the snapshot whose states and histories the forward reads in place; lu[6] = the
    // state rows every branch of a tree forward shares (attention's shared prefix past P)
    const uint32_t v[8] = {(uint32_t)n, (uint32_t)P, SD_CONTEXT, has_cache ? 1u : 0u, chunks, nseq, tree, 0u};
    std::memcpy(up_h, v, sizeof(v));
    const void* prefix = cache ? cache->arena : nullptr;
    std::memcpy(up_h + LU_PREFIX_BYTE, &prefix, sizeof(prefix));
    std::memcpy(up_h + pool.off_ids, ids, n * 4);
    uint32_t* rows_h = reinterpret_cast<uint32_t*>(up_h + pool.off_rows);
    for (size_t r = 0; r < n_rows; r++) rows_h[r] = (uint32_t)rows[r];
    const size_t end = std::max(up_dirty, n_rows ? pool.off_rows + n_rows * 4 : pool.off_ids + n * 4);
    SD_HIP(hipMemcpyAsync(lu, up_h, end, hipMemcpyHostToDevice, st));
    up_dirty = 0;
}

// Restore (src/engine.rs:552-571).  The GDN states and conv histories are not copied: the kernels
// read them from the snapshot in place (upload puts its address in the lu block) and write the live
// arena.  The K/V prefix rows are copied only when the live cache does not already hold this
// snapshot's prefix (question forwards write rows >= P only, so after one restore the prefix stays
// valid for every later question).
void Engine::restore(const Snapshot* cache, size_t P) {
    if (cache) {
        std::vector<CopyDesc> cp;
        if (kv_owner != cache->id) {
            // K and V^T in 32-key blocks (the attention kernel's layouts, one kv head's first P32 keys
            // contiguous), whole blocks: the live rows P..P32-1 are rewritten by the forward before
            // any read (a forward writes rows >= P of its own ids first) or lie past every key it reads
            const size_t row = (size_t)cfg.hd * 2, P32 = (P + 31) & ~size_t(31);
            for (size_t a = 0; a < attn_layers.size(); a++) {
                const LayerW& W = layers[attn_layers[a]];
                cp.push_back(CopyDesc{cache->kv(a, 0), reinterpret_cast<uint8_t*>(W.kc), (uint64_t)cfg.hk, P32 * row,
                                      P32 * row, SD_CONTEXT * row});
                cp.push_back(CopyDesc{cache->kv(a, 1), reinterpret_cast<uint8_t*>(W.vc), (uint64_t)cfg.hk, P32 * row,
                                      P32 * row, SD_CONTEXT * row});
            }
            kv_owner = cache->id;
        }
        if (!cp.empty()) copy_batch(cp.data(), cp.size(), st);
    } else {
        fill_u32(reinterpret_cast<uint32_t*>(arena + arena_state_bytes), (arena_bytes - arena_state_bytes) / 4, 0u, st);
        kv_owner = 0;
    }
}

void Engine::run_checked(Plan& pl) {
    std::vector<float> xh;
    for (size_t i = 0; i < pl.steps.size(); i++) {
        const Step& s = pl.steps[i];
        s.run(st);
        const hipError_t se = hipStreamSynchronize(st);
        const hipError_t le = hipGetLastError();
        if (se != hipSuccess || le != hipSuccess)
            throw Error("checked forward: step " + std::to_string(i) + " (" + s.label + "): " +
                        hipGetErrorString(se != hipSuccess ? se : le));
        if (std::strcmp(s.label, "norm") != 0) continue;
        xh.resize((size_t)pl.L * cfg.d);
        SD_HIP(hipMemcpy(xh.data(), pool.x, xh.size() * 4, hipMemcpyDeviceToHost));
        for (size_t e = 0; e < xh.size(); e++)
            if (!std::isfinite(xh[e]))
                throw Error("checked forward: step " + std::to_string(i) + " (norm): the residual stream holds a "
                            "non-finite value at row " + std::to_string(e / cfg.d) + ", column " +
                            std::to_string(e % cfg.d));
    }
}

void Engine::launch_and_read(Plan& pl, size_t n_rows, bool timed, bool read) {
    if (timed) SD_HIP(hipEventRecord(ev0, st));
    if (checked) {
        run_checked(pl);
    } else if (pl.exec) {
        SD_HIP(hipGraphLaunch(pl.exec, st));
    } else {
        for (auto& s : pl.steps) s.run(st);
    }
    if (n_rows) {
        // a compact plan's read rows are already gathered, in row order, in pool.xc
        SD_CHECK(!pl.compact || (size_t)pl.compact == n_rows, "compact plan run with another row count");
        if (pl.compact) add_norm(pool.xc, pl.last_y, final_norm, cfg.d, nullptr, (int)n_rows, nullptr, pool.out, st);
        else add_norm(pool.x, pl.last_y, final_norm, cfg.d, pool.rows, (int)n_rows, nullptr, pool.out, st);
    }
    if (!read) return;
    if (timed) SD_HIP(hipEventRecord(ev1, st));
    if (n_rows) SD_HIP(hipMemcpyAsync(out_h, pool.out, n_rows * cfg.d * 4, hipMemcpyDeviceToHost, st));
}

void Engine::finish(size_t n_rows, float* hidden, bool timed, double* gpu_ms) {
    if (n_rows) {
        std::memcpy(hidden, out_h, n_rows * cfg.d * 4);
        // A rotated torso: the head's basis is unrotate * FWHT(row) (src/engine.rs:652-660).
        if (!unrotate.empty())
            for (size_t r = 0; r < n_rows; r++) {
                float* x = hidden + r * cfg.d;
                fwht(x, cfg.d);
                for (int j = 0; j < cfg.d; j++) x[j] = (float)((double)x[j] * unrotate[j]);
            }
    }
    if (gpu_ms) {
        *gpu_ms = NAN;
        if (timed) {
            float ms = 0.f;
            SD_HIP(hipEventElapsedTime(&ms, ev0, ev1));
            *gpu_ms = ms;
        }
    }
}

void Engine::forward(const uint32_t* ids, size_t n, const size_t* rows, size_t n_rows, const Snapshot* cache,
                     bool keep, bool timed, float* hidden, double* gpu_ms, Snapshot** snap_out) {
    const size_t P = cache ? cache->len : 0;
    if (n == 0 || P + n > SD_CONTEXT)
        throw Error("context of " + std::to_string(P + n) + " tokens: must be 1 to " + std::to_string(SD_CONTEXT));
    for (size_t r = 0; r < n_rows; r++)
        if (rows[r] >= n) throw Error("row " + std::to_string(rows[r]) + " out of range for " + std::to_string(n) + " tokens");
    if (cache && cache->engine != this) throw Error("snapshot belongs to another engine");
    for (uint32_t i = 0; i < n; i++)
        if (ids[i] >= (uint32_t)vocab) throw Error("token id " + std::to_string(ids[i]) + " out of range for vocab " + std::to_string(vocab));
    const int L = (int)n;
    SD_CHECK(n_rows <= SD_CONTEXT, "at most 4096 hidden rows per forward");
    ensure_pool(std::max(L, (int)n_rows));  // the row tables and outputs hold n_rows entries
    Plan& pl = plan(L, 0, false, 0, n_rows == 0, (int)n_rows);
    upload(ids, n, rows, n_rows, P, cache != nullptr, 0, 0, cache);
    restore(cache, P);
    launch_and_read(pl, n_rows, timed);
    Snapshot* snap = nullptr;
    if (keep) {
        const size_t T = P + n;
        snap = new Snapshot();
        snap->engine = this;
        snap->len = T;
        snap->id = ++snapshot_ids;
        const size_t T32 = (T + 31) & ~size_t(31);
        snap->kv_stride = (size_t)cfg.hk * T32 * cfg.hd * 2;
        snap->arena_bytes = arena_bytes;
        snap->alloc_bytes = arena_bytes + attn_layers.size() * 2 * snap->kv_stride;
        try {
            snap->arena = snap_alloc(snap->alloc_bytes);
        } catch (...) {
            delete snap;
            throw;
        }
        // the arena image, then the K and V^T blocks of the first T32 keys of each kv head (whole 32-key
        // blocks; the keys past T are not read back)
        std::vector<CopyDesc> cp;
        cp.push_back(CopyDesc{arena, static_cast<uint8_t*>(snap->arena), 1, arena_bytes, arena_bytes, arena_bytes});
        const size_t row = (size_t)cfg.hd * 2;
        for (size_t a = 0; a < attn_layers.size(); a++) {
            const LayerW& W = layers[attn_layers[a]];
            cp.push_back(CopyDesc{reinterpret_cast<const uint8_t*>(W.kc), snap->kv(a, 0), (uint64_t)cfg.hk, T32 * row,
                                  SD_CONTEXT * row, T32 * row});
            cp.push_back(CopyDesc{reinterpret_cast<const uint8_t*>(W.vc), snap->kv(a, 1), (uint64_t)cfg.hk, T32 * row,
                                  SD_CONTEXT * row, T32 * row});
        }
        copy_batch(cp.data(), cp.size(), st);
        kv_owner = snap->id;
    }
    const hipError_t se = hipStreamSynchronize(st);
    if (se != hipSuccess) {
        delete snap;
        throw Error(std::string("GPU: ") + hipGetErrorString(se));
    }
    finish(n_rows, hidden, timed, gpu_ms);
    if (snap_out) *snap_out = snap;
    else delete snap;
}

Plan& Engine::prepare_batch(const uint32_t* ids, const size_t* lens, size_t nseq, const size_t* rows, size_t n_rows,
                            const Snapshot* cache) {
    if (nseq == 0 || nseq > (size_t)SD_MAX_SEQS)
        throw Error("a batch holds 1 to " + std::to_string(SD_MAX_SEQS) + " sequences");
    size_t n = 0;
    bool any_short = false, any_long = false;
    for (size_t q = 0; q < nseq; q++) {
        if (lens[q] == 0) throw Error("sequence " + std::to_string(q) + " has no tokens");
        n += lens[q];
        (lens[q] <= 20 ? any_short : any_long) = true;
    }
    if (any_short && any_long)
        throw Error("a batch mixes sequences of at most 20 tokens with longer ones (their matmuls differ)");
    const size_t P = cache ? cache->len : 0;
    if (P + n > SD_CONTEXT)
        throw Error("context of " + std::to_string(P + n) + " tokens (prefix + every sequence): must be at most " +
                    std::to_string(SD_CONTEXT));
    for (size_t r = 0; r < n_rows; r++)
        if (rows[r] >= n) throw Error("row " + std::to_string(rows[r]) + " out of range for " + std::to_string(n) + " tokens");
    if (cache && cache->engine != this) throw Error("snapshot belongs to another engine");
    for (size_t i = 0; i < n; i++)
        if (ids[i] >= (uint32_t)vocab) throw Error("token id " + std::to_string(ids[i]) + " out of range for vocab " + std::to_string(vocab));
    const int L = (int)n;
    SD_CHECK(n_rows <= SD_CONTEXT, "at most 4096 hidden rows per forward");
    ensure_pool(std::max(L, (int)n_rows));  // the row tables and outputs hold n_rows entries
    Plan& pl = plan(L, (int)nseq, any_short, 0, false, (int)n_rows);
    // sequence tables (see Segs): rows, chunks of <= 64 rows inside each sequence, sequences
    uint32_t* rowt = reinterpret_cast<uint32_t*>(up_h + pool.off_seg_row);
    uint32_t* chunkt = reinterpret_cast<uint32_t*>(up_h + pool.off_seg_chunk);
    uint32_t nch = 0;
    size_t s0 = 0;
    std::vector<uint32_t> seqt(SD_MAX_SEQS + nseq);
    for (size_t q = 0; q < nseq; q++) {
        seqt[SD_MAX_SEQS + q] = (uint32_t)s0 | (uint32_t)(lens[q] << 16);
        for (size_t i = 0; i < lens[q]; i++) rowt[s0 + i] = (uint32_t)i | (uint32_t)(s0 << 16);
        const uint32_t first = nch;
        for (size_t k = 0; k < lens[q]; k += 64)
            chunkt[nch++] = (uint32_t)(s0 + k) | (uint32_t)(std::min<size_t>(64, lens[q] - k) << 16);
        seqt[q] = first | ((nch - first) << 16);
        s0 += lens[q];
    }
    SD_CHECK((int)nch <= pool.seg_chunk_cap, "forward_batch: chunk table overflow");
    std::memcpy(up_h + pool.off_seg_seq, seqt.data(), seqt.size() * 4);
    up_dirty = pool.off_seg_seq + seqt.size() * 4;  // sent with the ids by upload()
    upload(ids, n, rows, n_rows, P, cache != nullptr, nch, (uint32_t)nseq, cache);
    restore(cache, P);
    return pl;
}

void Engine::forward_batch(const uint32_t* ids, const size_t* lens, size_t nseq, const size_t* rows, size_t n_rows,
                           const Snapshot* cache, bool timed, float* hidden, double* gpu_ms) {
    Plan& pl = prepare_batch(ids, lens, nseq, rows, n_rows, cache);
    launch_and_read(pl, n_rows, timed);
    // The live K/V prefix rows are untouched (rows >= P only); the GDN state and history are not
    // meaningful after several sequences, and the next forward restores or clears them.
    const hipError_t se = hipStreamSynchronize(st);
    if (se != hipSuccess) throw Error(std::string("GPU: ") + hipGetErrorString(se));
    finish(n_rows, hidden, timed, gpu_ms);
}

void Engine::attach_head(const Head& head) {
    if (head_id == head.id) return;
    const size_t d = (size_t)cfg.d, dim = head.dim;
    if (head.t.at("norm.weight").size() != d || head.t.at("q.weight").size() != dim * d ||
        head.t.at("k.weight").size() != dim * d || head.t.at("q.bias").size() != dim || head.t.at("k.bias").size() != dim ||
        head.t.at("norm.bias").size() != d)
        throw Error("head: tensor shapes do not match hidden size " + std::to_string(d));
    if (head_dev) SD_HIP(hipFree(head_dev));
    head_dev = nullptr;
    head_id = 0;
    const char* names[6] = {"norm.weight", "norm.bias", "q.weight", "q.bias", "k.weight", "k.bias"};
    size_t off[7] = {0};
    for (int i = 0; i < 6; i++) off[i + 1] = off[i] + align256(head.t.at(names[i]).size() * 4);
    SD_HIP(hipMalloc(&head_dev, off[6]));
    const float* p[6];
    for (int i = 0; i < 6; i++) {
        const auto& v = head.t.at(names[i]);
        p[i] = reinterpret_cast<const float*>(static_cast<uint8_t*>(head_dev) + off[i]);
        SD_HIP(hipMemcpy(const_cast<float*>(p[i]), v.data(), v.size() * 4, hipMemcpyHostToDevice));
    }
    headw = HeadW{p[0], p[1], p[2], p[3], p[4], p[5], (int)dim};
    if (!unrotate.empty() && !unrot_dev) {
        unrot_dev = static_cast<double*>(dalloc(unrotate.size() * 8));
        SD_HIP(hipMemcpy(unrot_dev, unrotate.data(), unrotate.size() * 8, hipMemcpyHostToDevice));
    }
    head_id = head.id;
}

void Engine::ensure_head_bufs(size_t rows, size_t nq) {
    if (hb.rows >= rows && hb.nq >= nq && hb.dim == (size_t)headw.dim) return;
    rows = std::max(rows, std::max<size_t>(hb.rows, 64));
    nq = std::max(nq, std::max<size_t>(hb.nq, 32));
    if (hb.dev) SD_HIP(hipFree(hb.dev));
    if (hb.host) SD_HIP(hipHostFree(hb.host));
    hb = HeadBufs{};
    const size_t dim = (size_t)std::max(headw.dim, 1);
    // device: proj [rows][dim] | scale [nq] | probs [rows] | qtab [nq] | ooff [nq] | is_answer [rows]
    const size_t o1 = align256(rows * dim * 8), o2 = o1 + align256(nq * 8), o3 = o2 + align256(rows * 8),
                 o4 = o3 + align256(nq * 4), o5 = o4 + align256(nq * 4), o6 = o5 + align256(rows);
    SD_HIP(hipMalloc(&hb.dev, o6));
    uint8_t* d = static_cast<uint8_t*>(hb.dev);
    hb.proj = reinterpret_cast<double*>(d);
    hb.scale = reinterpret_cast<double*>(d + o1);
    hb.probs = reinterpret_cast<double*>(d + o2);
    hb.qtab = reinterpret_cast<uint32_t*>(d + o3);
    hb.ooff = reinterpret_cast<uint32_t*>(d + o4);
    hb.is_answer = d + o5;
    // host: scale | probs | qtab | ooff | is_answer (the same order as on the device, from scale)
    const size_t hbytes = o6 - o1;
    SD_HIP(hipHostMalloc(&hb.host, hbytes, hipHostMallocDefault));
    uint8_t* h = static_cast<uint8_t*>(hb.host);
    hb.scale_h = reinterpret_cast<double*>(h);
    hb.probs_h = reinterpret_cast<double*>(h + (o2 - o1));
    hb.qtab_h = reinterpret_cast<uint32_t*>(h + (o3 - o1));
    hb.ooff_h = reinterpret_cast<uint32_t*>(h + (o4 - o1));
    hb.is_answer_h = h + (o5 - o1);
    hb.rows = rows;
    hb.nq = nq;
    hb.dim = dim;
}

void Engine::ask_batch(const Head& head, const uint32_t* ids, const size_t* lens, size_t nseq, const size_t* rows,
                       const size_t* n_opts, const double* temps, const Snapshot* cache, bool timed, double* probs,
                       double* gpu_ms) {
    size_t n_rows = 0, n_prob = 0;
    for (size_t q = 0; q < nseq; q++) {
        if (n_opts[q] == 0) throw Error("question " + std::to_string(q) + " has no options");
        n_rows += n_opts[q] + 1;
        n_prob += n_opts[q];
    }
    SD_CHECK(n_rows < 65536, "ask_batch: too many rows");
    attach_head(head);
    Plan& pl = prepare_batch(ids, lens, nseq, rows, n_rows, cache);
    ask_tail(pl, nseq, n_opts, temps, n_rows, n_prob, timed, probs, gpu_ms);
}

void Engine::ask_tail(Plan& pl, size_t nseq, const size_t* n_opts, const double* temps, size_t n_rows, size_t n_prob,
                      bool timed, double* probs, double* gpu_ms) {
    ensure_head_bufs(n_rows, nseq);
    size_t r = 0, o = 0;
    for (size_t q = 0; q < nseq; q++) {
        hb.qtab_h[q] = (uint32_t)r | (uint32_t)(n_opts[q] << 16);
        hb.ooff_h[q] = (uint32_t)o;
        hb.scale_h[q] = std::pow((double)headw.dim, -0.5) / std::max(temps[q], 1e-6);
        for (size_t k = 0; k < n_opts[q]; k++) hb.is_answer_h[r + k] = 0;
        hb.is_answer_h[r + n_opts[q]] = 1;
        r += n_opts[q] + 1;
        o += n_opts[q];
    }
    // the tables: scale .. is_answer are one contiguous span on both sides
    const size_t span = static_cast<size_t>(reinterpret_cast<uint8_t*>(hb.is_answer) + n_rows -
                                            reinterpret_cast<uint8_t*>(hb.scale));
    SD_HIP(hipMemcpyAsync(hb.scale, hb.scale_h, span, hipMemcpyHostToDevice, st));
    launch_and_read(pl, n_rows, timed, false);
    if (!unrotate.empty()) unrotate_rows(pool.out, (int)n_rows, cfg.d, unrot_dev, st);
    head_rows(pool.out, (int)n_rows, cfg.d, headw, hb.is_answer, hb.proj, st);
    head_probs(hb.proj, headw.dim, hb.qtab, hb.scale, hb.ooff, (int)nseq, hb.probs, st);
    if (timed) SD_HIP(hipEventRecord(ev1, st));
    SD_HIP(hipMemcpyAsync(hb.probs_h, hb.probs, n_prob * 8, hipMemcpyDeviceToHost, st));
    const hipError_t se = hipStreamSynchronize(st);
    if (se != hipSuccess) throw Error(std::string("GPU: ") + hipGetErrorString(se));
    std::memcpy(probs, hb.probs_h, n_prob * 8);
    finish(0, nullptr, timed, gpu_ms);
}

void Engine::ask_tree(const Head& head, const uint32_t* state, size_t n_state, const uint32_t* ids, const size_t* lens,
                      size_t nq, const size_t* rows, const size_t* n_opts, const double* temps, bool timed,
                      double* probs, double* gpu_ms) {
    if (nq == 0 || nq + 1 > (size_t)SD_MAX_SEQS)
        throw Error("a tree forward holds 1 to " + std::to_string(SD_MAX_SEQS - 1) + " questions");
    if (n_state == 0) throw Error("context of 0 tokens: must be 1 to " + std::to_string(SD_CONTEXT));
    size_t nb = 0, n_rows = 0, n_prob = 0;
    for (size_t q = 0; q < nq; q++) {
        // the questions' matmuls must be the tiled kernels' (f16 dequant) as in their own forwards
        if (lens[q] <= 20) throw Error("a tree forward needs questions of more than 20 tokens");
        if (n_opts[q] == 0) throw Error("question " + std::to_string(q) + " has no options");
        nb += lens[q];
        n_rows += n_opts[q] + 1;
        n_prob += n_opts[q];
    }
    SD_CHECK(n_rows < 65536, "ask_tree: too many rows");
    const size_t n = n_state + nb;
    if (n > SD_CONTEXT)
        throw Error("context of " + std::to_string(n) + " tokens (state + every question): must be at most " +
                    std::to_string(SD_CONTEXT));
    for (size_t r = 0; r < n_rows; r++)
        if (rows[r] >= nb) throw Error("row " + std::to_string(rows[r]) + " out of range for " + std::to_string(nb) + " tokens");
    for (size_t i = 0; i < n_state; i++)
        if (state[i] >= (uint32_t)vocab) throw Error("token id " + std::to_string(state[i]) + " out of range for vocab " + std::to_string(vocab));
    for (size_t i = 0; i < nb; i++)
        if (ids[i] >= (uint32_t)vocab) throw Error("token id " + std::to_string(ids[i]) + " out of range for vocab " + std::to_string(vocab));
    attach_head(head);
    const int L = (int)n, S = (int)n_state, nseq = (int)nq + 1;
    ensure_pool(std::max(L, (int)n_rows));
    Plan& pl = plan(L, nseq, false, S, false, (int)n_rows);
    // Sequence tables (see Segs): sequence 0 the state, q + 1 question q.  A question row's index in
    // its sequence is S + its own index (its RoPE position); its sequence starts at its first row.
    uint32_t* rowt = reinterpret_cast<uint32_t*>(up_h + pool.off_seg_row);
    uint32_t* chunkt = reinterpret_cast<uint32_t*>(up_h + pool.off_seg_chunk);
    std::vector<uint32_t> seqt(SD_MAX_SEQS + nseq);
    uint32_t nch = 0;
    size_t s0 = 0;
    for (int q = 0; q < nseq; q++) {
        const size_t len = q == 0 ? n_state : lens[q - 1];
        const size_t base = q == 0 ? 0 : n_state;
        seqt[SD_MAX_SEQS + q] = (uint32_t)s0 | (uint32_t)(len << 16);
        for (size_t i = 0; i < len; i++) rowt[s0 + i] = (uint32_t)(base + i) | (uint32_t)(s0 << 16);
        const uint32_t first = nch;
        for (size_t k = 0; k < len; k += 64)
            chunkt[nch++] = (uint32_t)(s0 + k) | (uint32_t)(std::min<size_t>(64, len - k) << 16);
        seqt[q] = first | ((nch - first) << 16);
        s0 += len;
    }
    SD_CHECK((int)nch <= pool.seg_chunk_cap, "ask_tree: chunk table overflow");
    std::memcpy(up_h + pool.off_seg_seq, seqt.data(), seqt.size() * 4);
    up_dirty = pool.off_seg_seq + seqt.size() * 4;  // sent with the ids by upload()
    std::vector<uint32_t> all(state, state + n_state);
    all.insert(all.end(), ids, ids + nb);
    std::vector<size_t> grows(rows, rows + n_rows);
    for (size_t& r : grows) r += n_state;
    // has_cache set with no snapshot named: the branches' delta rule starts from the live state and
    // history, which the state's scan writes earlier in the same forward
    upload(all.data(), n, grows.data(), n_rows, 0, true, nch, (uint32_t)nseq, nullptr, (uint32_t)S);
    restore(nullptr, 0);  // the state starts from a cleared history (the live state is overwritten)
    ask_tail(pl, nq, n_opts, temps, n_rows, n_prob, timed, probs, gpu_ms);
}

std::vector<std::pair<const char*, double>> Engine::profile(const uint32_t* ids, size_t n) {
    if (n == 0 || n > SD_CONTEXT) throw Error("profiling needs 1 to 4096 tokens");
    for (uint32_t i = 0; i < n; i++)
        if (ids[i] >= (uint32_t)vocab) throw Error("token id out of range");
    const int L = (int)n;
    ensure_pool(L);
    Plan& pl = plan(L);
    upload(ids, n, nullptr, 0, 0, false, 0, 0, nullptr);
    restore(nullptr, 0);
    // A step that launched a GEMM is timed by the kernel's own start and end; any other step by
    // the events recorded between steps.
    const size_t ns = pl.steps.size();
    std::vector<hipEvent_t> evs(ns + 1), kev(2 * ns);
    std::vector<int> own(ns, 0);
    for (auto& e : evs) SD_HIP(hipEventCreate(&e));
    for (auto& e : kev) SD_HIP(hipEventCreate(&e));
    struct Reset {
        ~Reset() { kernel_events() = nullptr; }
    } reset;
    SD_HIP(hipEventRecord(evs[0], st));
    for (size_t i = 0; i < ns; i++) {
        KernelEvents ke{kev[2 * i], kev[2 * i + 1], 0};
        kernel_events() = &ke;
        pl.steps[i].run(st);
        kernel_events() = nullptr;
        own[i] = ke.launches;
        SD_HIP(hipEventRecord(evs[i + 1], st));
    }
    SD_HIP(hipStreamSynchronize(st));
    std::vector<std::pair<const char*, double>> by;
    for (size_t i = 0; i < ns; i++) {
        float ms = 0.f;
        if (own[i]) SD_HIP(hipEventElapsedTime(&ms, kev[2 * i], kev[2 * i + 1]));
        else SD_HIP(hipEventElapsedTime(&ms, evs[i], evs[i + 1]));
        auto f = std::find_if(by.begin(), by.end(), [&](auto& p) { return std::strcmp(p.first, pl.steps[i].label) == 0; });
        if (f == by.end()) by.emplace_back(pl.steps[i].label, ms);
        else f->second += ms;
    }
    for (auto& e : evs) (void)hipEventDestroy(e);
    for (auto& e : kev) (void)hipEventDestroy(e);
    std::sort(by.begin(), by.end(), [](auto& a, auto& b) { return a.second > b.second; });
    return by;
}

size_t Engine::trace(const uint32_t* ids, size_t n, const Snapshot* cache, const size_t* rows, size_t n_rows,
                     float* x_out, uint16_t* h_out, size_t cap) {
    const size_t P = cache ? cache->len : 0;
    if (n == 0 || P + n > SD_CONTEXT)
        throw Error("context of " + std::to_string(P + n) + " tokens: must be 1 to " + std::to_string(SD_CONTEXT));
    if (cache && cache->engine != this) throw Error("snapshot belongs to another engine");
    for (size_t i = 0; i < n; i++)
        if (ids[i] >= (uint32_t)vocab) throw Error("token id " + std::to_string(ids[i]) + " out of range for vocab " + std::to_string(vocab));
    for (size_t r = 0; r < n_rows; r++)
        if (rows[r] >= n) throw Error("row " + std::to_string(rows[r]) + " out of range for " + std::to_string(n) + " tokens");
    const int L = (int)n;
    ensure_pool(L);
    Plan& pl = plan(L);
    upload(ids, n, nullptr, 0, P, cache != nullptr, 0, 0, cache);
    restore(cache, P);
    const size_t d = (size_t)cfg.d;
    size_t taps = 0;
    for (auto& step : pl.steps) {
        step.run(st);
        if (std::strcmp(step.label, "norm") != 0) continue;
        if (taps < cap) {
            SD_HIP(hipStreamSynchronize(st));
            for (size_t r = 0; r < n_rows; r++) {
                SD_HIP(hipMemcpy(x_out + (taps * n_rows + r) * d, pool.x + rows[r] * d, d * 4, hipMemcpyDeviceToHost));
                SD_HIP(hipMemcpy(h_out + (taps * n_rows + r) * d, pool.h + rows[r] * d, d * 2, hipMemcpyDeviceToHost));
            }
        }
        taps++;
    }
    SD_HIP(hipStreamSynchronize(st));
    return taps;
}

Snapshot::~Snapshot() {
    if (!arena) return;
    if (engine) engine->snap_release(arena, alloc_bytes);
    else (void)hipFree(arena);
}

}  // namespace sd
