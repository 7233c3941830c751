// The pointer head on the CPU in f64 (reference: src/head.rs): LayerNorm (eps 1e-5), q from the
// answer row, k from each option row, logits = k.q * dim^-0.5 / max(T, 1e-6), softmax.  Loaded
// from head.safetensors (8-byte header length, JSON header, raw little-endian F32 data).
#include "head.h"

#include <atomic>
#include <cmath>
#include <cstring>

#include <immintrin.h>

namespace sd {
namespace {

// Minimal JSON reader for the safetensors header: objects, arrays, strings, numbers, literals.
struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    double num = 0;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
    const JVal* get(const char* k) const {
        for (auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct JParser {
    const char* p;
    const char* end;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
    }
    bool lit(const char* s) {
        const size_t n = std::strlen(s);
        if ((size_t)(end - p) >= n && std::memcmp(p, s, n) == 0) {
            p += n;
            return true;
        }
        return false;
    }
    std::string string() {
        if (p >= end || *p != '"') throw Error("head.safetensors: malformed");
        p++;
        std::string out;
        while (p < end && *p != '"') {
            if (*p == '\\') {
                p++;
                if (p >= end) break;
                const char c = *p++;
                switch (c) {
                    case 'n': out += '\n'; break;
                    case 't': out += '\t'; break;
                    case 'r': out += '\r'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'u':
                        if (end - p < 4) throw Error("head.safetensors: malformed");
                        out += '?';  // names here are ASCII; any escape is kept as a placeholder
                        p += 4;
                        break;
                    default: out += c;
                }
            } else {
                out += *p++;
            }
        }
        if (p >= end) throw Error("head.safetensors: malformed");
        p++;
        return out;
    }
    JVal value(int depth = 0) {
        if (depth > 64) throw Error("head.safetensors: malformed");
        ws();
        JVal v;
        if (p >= end) throw Error("head.safetensors: malformed");
        if (*p == '{') {
            v.kind = JVal::Obj;
            p++;
            ws();
            if (p < end && *p == '}') {
                p++;
                return v;
            }
            for (;;) {
                ws();
                std::string k = string();
                ws();
                if (p >= end || *p != ':') throw Error("head.safetensors: malformed");
                p++;
                v.obj.emplace_back(std::move(k), value(depth + 1));
                ws();
                if (p < end && *p == ',') {
                    p++;
                    continue;
                }
                if (p < end && *p == '}') {
                    p++;
                    return v;
                }
                throw Error("head.safetensors: malformed");
            }
        }
        if (*p == '[') {
            v.kind = JVal::Arr;
            p++;
            ws();
            if (p < end && *p == ']') {
                p++;
                return v;
            }
            for (;;) {
                v.arr.push_back(value(depth + 1));
                ws();
                if (p < end && *p == ',') {
                    p++;
                    continue;
                }
                if (p < end && *p == ']') {
                    p++;
                    return v;
                }
                throw Error("head.safetensors: malformed");
            }
        }
        if (*p == '"') {
            v.kind = JVal::Str;
            v.str = string();
            return v;
        }
        if (lit("true")) {
            v.kind = JVal::Bool;
            v.num = 1;
            return v;
        }
        if (lit("false")) {
            v.kind = JVal::Bool;
            return v;
        }
        if (lit("null")) return v;
        char* e = nullptr;
        v.num = std::strtod(p, &e);
        if (e == p || e > end) throw Error("head.safetensors: malformed");
        v.kind = JVal::Num;
        p = e;
        return v;
    }
};

}  // namespace

void Head::load(const uint8_t* bytes, size_t len) {
    static std::atomic<uint64_t> ids{0};
    id = ++ids;
    if (len < 8) throw Error("head.safetensors: malformed");
    uint64_t n = 0;
    std::memcpy(&n, bytes, 8);
    if (n > len - 8) throw Error("head.safetensors: malformed");
    std::string header(reinterpret_cast<const char*>(bytes) + 8, (size_t)n);
    JParser jp{header.c_str(), header.c_str() + header.size()};
    const JVal root = jp.value();
    if (root.kind != JVal::Obj) throw Error("head.safetensors: malformed");
    const uint8_t* data = bytes + 8 + n;
    const size_t dlen = len - 8 - (size_t)n;
    for (auto& kv : root.obj) {
        if (kv.first == "__metadata__") continue;
        const JVal& e = kv.second;
        const JVal* dt = e.get("dtype");
        const JVal* shape = e.get("shape");
        const JVal* offs = e.get("data_offsets");
        if (!dt || dt->kind != JVal::Str || !shape || shape->kind != JVal::Arr || !offs || offs->kind != JVal::Arr ||
            offs->arr.size() != 2)
            throw Error("head.safetensors: malformed");
        if (dt->str != "F32") throw Error("head tensor " + kv.first + " is " + dt->str + ", expected F32");
        const size_t a = (size_t)offs->arr[0].num, b = (size_t)offs->arr[1].num;
        if (a > b || b > dlen || (b - a) % 4) throw Error("head.safetensors: malformed");
        if (kv.first == "q.weight" && !shape->arr.empty()) dim = (size_t)shape->arr[0].num;
        std::vector<float> v((b - a) / 4);
        std::memcpy(v.data(), data + a, b - a);
        t[kv.first] = std::move(v);
    }
    for (const char* k : {"norm.weight", "norm.bias", "q.weight", "q.bias", "k.weight", "k.bias"})
        if (!t.count(k)) throw Error(std::string("head.safetensors: no ") + k);
}

std::vector<double> Head::normalize(const float* x, size_t d) const {
    double mean = 0;
    for (size_t j = 0; j < d; j++) mean += (double)x[j];
    mean /= (double)d;
    double var = 0;
    for (size_t j = 0; j < d; j++) var += ((double)x[j] - mean) * ((double)x[j] - mean);
    var /= (double)d;
    const double r = 1.0 / std::sqrt(var + 1e-5);
    const auto& nw = t.at("norm.weight");
    const auto& nb = t.at("norm.bias");
    std::vector<double> xn(d);
    for (size_t j = 0; j < d; j++) xn[j] = ((double)x[j] - mean) * r * (double)nw[j] + (double)nb[j];
    return xn;
}

// f64 dot product of f32 weights with f64 values; with AVX2 + FMA when the host has them (four
// 4-wide partial sums).  The reference widens to f64 and sums in f64 too; the summation order only
// moves the last bits.
__attribute__((target("avx2,fma"))) static double dot_avx2(const float* a, const double* b, size_t n) {
    __m256d s0 = _mm256_setzero_pd(), s1 = _mm256_setzero_pd(), s2 = _mm256_setzero_pd(), s3 = _mm256_setzero_pd();
    size_t j = 0;
    for (; j + 16 <= n; j += 16) {
        s0 = _mm256_fmadd_pd(_mm256_cvtps_pd(_mm_loadu_ps(a + j)), _mm256_loadu_pd(b + j), s0);
        s1 = _mm256_fmadd_pd(_mm256_cvtps_pd(_mm_loadu_ps(a + j + 4)), _mm256_loadu_pd(b + j + 4), s1);
        s2 = _mm256_fmadd_pd(_mm256_cvtps_pd(_mm_loadu_ps(a + j + 8)), _mm256_loadu_pd(b + j + 8), s2);
        s3 = _mm256_fmadd_pd(_mm256_cvtps_pd(_mm_loadu_ps(a + j + 12)), _mm256_loadu_pd(b + j + 12), s3);
    }
    const __m256d s = _mm256_add_pd(_mm256_add_pd(s0, s1), _mm256_add_pd(s2, s3));
    double v[4];
    _mm256_storeu_pd(v, s);
    double r = (v[0] + v[1]) + (v[2] + v[3]);
    for (; j < n; j++) r += (double)a[j] * b[j];
    return r;
}

static double dot_plain(const float* a, const double* b, size_t n) {
    double s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t j = 0;
    for (; j + 8 <= n; j += 8)
        for (int u = 0; u < 8; u++) s[u] += (double)a[j + u] * b[j + u];
    for (; j < n; j++) s[0] += (double)a[j] * b[j];
    return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

static double dot(const float* a, const double* b, size_t n) {
    static const bool avx2 = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    return avx2 ? dot_avx2(a, b, n) : dot_plain(a, b, n);
}

// out[r][o] = bias[o] + W[o] . xs[r] in f64.  Each weight row is read once for all rows; the dot
std::vector<std::vector<double>> Head::project(const char* which, const std::vector<std::vector<double>>& xs,
                                               size_t d) const {
    const auto& w = t.at(std::string(which) + ".weight");
    const auto& b = t.at(std::string(which) + ".bias");
    std::vector<std::vector<double>> out(xs.size(), std::vector<double>(dim));
    for (size_t o = 0; o < dim; o++) {
        const float* wr = w.data() + o * d;
        for (size_t r = 0; r < xs.size(); r++) out[r][o] = (double)b[o] + dot(wr, xs[r].data(), d);
    }
    return out;
}

std::vector<double> Head::probs(const float* hidden, size_t n_rows, size_t d, double temperature) const {
    if (n_rows < 2) throw Error("head: need at least one option row and the answer row");
    if (t.at("norm.weight").size() != d || t.at("q.weight").size() != dim * d || t.at("k.weight").size() != dim * d)
        throw Error("head: tensor shapes do not match hidden size " + std::to_string(d));
    std::vector<std::vector<double>> opts;
    for (size_t i = 0; i + 1 < n_rows; i++) opts.push_back(normalize(hidden + i * d, d));
    const std::vector<double> q = project("q", {normalize(hidden + (n_rows - 1) * d, d)}, d)[0];
    const std::vector<std::vector<double>> k = project("k", opts, d);
    const double scale = std::pow((double)dim, -0.5) / std::max(temperature, 1e-6);
    std::vector<double> logits(n_rows - 1);
    for (size_t i = 0; i + 1 < n_rows; i++) {
        double s = 0;
        for (size_t o = 0; o < dim; o++) s += k[i][o] * q[o];
        logits[i] = s * scale;
    }
    double mx = -INFINITY;
    for (double l : logits) mx = std::max(mx, l);
    double z = 0;
    for (double& l : logits) z += (l = std::exp(l - mx));
    for (double& l : logits) l /= z;
    return logits;
}

}  // namespace sd
