/*
 * CPU oracle for the strands-decider torso.  TEST INFRASTRUCTURE ONLY: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only as
 * the checker or the timed CPU baseline.  The product (libsdhip.so) never calls it.
 *
 * Every function restates one WGSL kernel of the reference engine (mircodz/strands-decider-rs,
 * src/kernels.rs) with the same rounding points: f16 storage where the WGSL stores f16, f32
 * arithmetic where the WGSL computes in f32.  Reductions use f32 (or f64 where marked) in a fixed
 * order; the reference's own order depends on the GPU's subgroup width, so only rounding-level
 * agreement is expected.  f16 conversions are software round-to-nearest-even (no _Float16 in gcc 11
 * on x86-64); they are pinned exhaustively against numpy.float16 by tests/test_oracle.py.
 *
 * Pinning of each function (what checks it independently of this file) is listed in
 * tests/test_oracle.py; the one restated function with no independent check is marked
 * "parity unpinned" below (none at present).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- f16 <-> f32 ------------------------------------------------------------------------ */

float or_h2f(uint16_t h) {
    uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 31u, m = h & 1023u;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 1024u), (int)e - 25);
    return s ? -v : v;
}

uint16_t or_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                  /* f16 subnormal range */
        float a;
        memcpy(&a, &ax, 4);
        uint32_t r = (uint32_t)nearbyintf(a * 16777216.0f); /* exact scaling; RNE */
        return (uint16_t)(sign | r);
    }
    uint32_t e = (ax >> 23) - 127u + 15u, m = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13), rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

void or_h2f_n(const uint16_t* h, float* f, int64_t n) {
    for (int64_t i = 0; i < n; i++) f[i] = or_h2f(h[i]);
}

void or_f2h_n(const float* f, uint16_t* h, int64_t n) {
    for (int64_t i = 0; i < n; i++) h[i] = or_f2h(f[i]);
}

static inline float rnd16(float f) { return or_h2f(or_f2h(f)); }

/* ---- quantized values (src/kernels.rs:63-89 embed, 550-576 decode_from) ------------------ */

/* Quant code of element e (0..31) of block `blk`. */
static inline uint32_t qcode(const uint32_t* Q, int64_t blk, int e, int bits) {
    if (bits == 4) return (Q[blk * 4 + e / 8] >> (4 * (e % 8))) & 15u;
    uint32_t lo = (Q[blk * bits + e / 16] >> (2 * (e % 16))) & 3u;
    if (bits == 3) lo |= ((Q[blk * 3 + 2] >> e) & 1u) << 2;
    return lo;
}

/* ids -> x (f32 [L, d]); src/kernels.rs:63-89.  Bi is NULL for symmetric formats. */
void or_embed(const uint32_t* ids, int L, const uint32_t* Q, const uint16_t* S, const uint16_t* Bi,
              int d, int bits, int group, int asym, float* x) {
    int nb = d / 32, gdiv = group / 32;
    for (int t = 0; t < L; t++) {
        for (int b = 0; b < nb; b++) {
            int64_t blk = (int64_t)ids[t] * nb + b;
            int64_t g = group == 32 ? blk : blk / gdiv;
            float sc = or_h2f(S[g]);
            float bi = asym ? or_h2f(Bi[g]) : 0.0f;
            for (int e = 0; e < 32; e++) {
                float q = (float)qcode(Q, blk, e, bits);
                x[(int64_t)t * d + b * 32 + e] = asym ? q * sc + bi : (q - (float)(1 << (bits - 1))) * sc;
            }
        }
    }
}

/* ---- matmul: Y[M,N] f16 = A[M,K] f16 . deq(W[N,K])^T ------------------------------------ */

/* Dequantize row n of W into w[K].  f16_deq: the tiled kernel's f16 dequant
 * ((f16(q) - 8) * sc rounded to f16, src/kernels.rs:668-672); else the GEMV's f32 dequant
 * (src/kernels.rs:572, 620; asym is fma(q, sc, bi) in f32). */
static void deq_row(const uint32_t* W, const uint16_t* Sc, const uint16_t* Bi, int64_t n, int K,
                    int bits, int group, int asym, int f16_deq, float* w) {
    int nb = K / 32, gdiv = group / 32;
    for (int b = 0; b < nb; b++) {
        int64_t blk = n * nb + b;
        int64_t g = group == 32 ? blk : blk / gdiv;
        float sc = or_h2f(Sc[g]);
        float bi = asym ? or_h2f(Bi[g]) : 0.0f;
        for (int e = 0; e < 32; e++) {
            float q = (float)qcode(W, blk, e, bits);
            float v = asym ? fmaf(q, sc, bi) : (q - (float)(1 << (bits - 1))) * sc;
            w[b * 32 + e] = f16_deq ? rnd16(v) : v;
        }
    }
}

/* The dequantized weights W[N][K] as f32 (each f16-representable when f16_deq). */
void or_dequant(const uint32_t* W, const uint16_t* Sc, const uint16_t* Bi, int N, int K, int bits, int group,
                int asym, int f16_deq, float* out) {
    for (int n = 0; n < N; n++) deq_row(W, Sc, Bi, n, K, bits, group, asym, f16_deq, out + (int64_t)n * K);
}

/* src/kernels.rs:590-709 (gemv and tiled): f32 accumulation, f16 output.  Bi may be NULL. */
void or_matmul(const uint16_t* A, const uint32_t* W, const uint16_t* Sc, const uint16_t* Bi, int M,
               int N, int K, int bits, int group, int asym, int f16_deq, uint16_t* Y) {
    float* Af = (float*)malloc(sizeof(float) * (size_t)M * K);
    or_h2f_n(A, Af, (int64_t)M * K);
#pragma omp parallel
    {
        float* w = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
        for (int n = 0; n < N; n++) {
            deq_row(W, Sc, Bi, n, K, bits, group, asym, f16_deq, w);
            for (int m = 0; m < M; m++) {
                const float* a = Af + (int64_t)m * K;
                float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (int k = 0; k < K; k += 8)
                    for (int j = 0; j < 8; j++) p[j] += a[k + j] * w[k + j];
                float acc = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
                Y[(int64_t)m * N + n] = or_f2h(acc);
            }
        }
        free(w);
    }
    free(Af);
}

/* ---- residual add + RMSNorm (src/kernels.rs:93-120) -------------------------------------- */

/* For r in 0..nrows: row = rows[r]; if y: x[row] += f32(y[row]) (x updated in place);
 * out[r] = x[row] * rsqrt(mean(x^2) + 1e-6) * w, as f16 (out16) or f32 (out32). */
void or_add_norm(float* x, const uint16_t* y, const float* w, int d, const uint32_t* rows, int nrows,
                 uint16_t* out16, float* out32) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < nrows; r++) {
        int64_t o = (int64_t)rows[r] * d;
        float ss = 0.0f;
        for (int c = 0; c < d; c++) {
            float a = x[o + c];
            if (y) {
                a += or_h2f(y[o + c]);
                x[o + c] = a;
            }
            ss += a * a;
        }
        float inv = 1.0f / sqrtf(ss / (float)d + 1e-6f);
        for (int c = 0; c < d; c++) {
            float v = x[o + c] * inv * w[c];
            if (out16) out16[(int64_t)r * d + c] = or_f2h(v);
            else out32[(int64_t)r * d + c] = v;
        }
    }
}

/* ---- elementwise ------------------------------------------------------------------------- */

/* mid[t, j] = f16(silu(g) * u), big[t] = [g (I) | u (I)]; src/kernels.rs:123-135. */
void or_silu_mul(const uint16_t* big, int L, int I, uint16_t* mid) {
    for (int64_t t = 0; t < L; t++)
        for (int j = 0; j < I; j++) {
            float g = or_h2f(big[t * 2 * I + j]), u = or_h2f(big[t * 2 * I + I + j]);
            mid[t * I + j] = or_f2h(g / (1.0f + expf(-g)) * u);
        }
}

/* y[t, j] = f16(f32(y) + c[j]); src/kernels.rs:138-149. */
void or_add_bias(uint16_t* y, int L, int N, const float* c) {
    for (int64_t t = 0; t < L; t++)
        for (int j = 0; j < N; j++) y[t * N + j] = or_f2h(or_h2f(y[t * N + j]) + c[j]);
}

/* Depthwise causal conv (k = 4) + SiLU; rows before t = 0 from hist [3][C];
 * src/kernels.rs:152-170.  w is [C][4] f32, out [L][C] f32. */
void or_conv(const uint16_t* big, int stride, int L, int C, const float* w, const uint16_t* hist, float* out) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < L; t++)
        for (int c = 0; c < C; c++) {
            float s = 0.0f;
            for (int j = 0; j < 4; j++) {
                int tt = t + j - 3;
                float v = tt >= 0 ? or_h2f(big[(int64_t)tt * stride + c]) : or_h2f(hist[(int64_t)(tt + 3) * C + c]);
                s += w[c * 4 + j] * v;
            }
            out[(int64_t)t * C + c] = s / (1.0f + expf(-s));
        }
}

/* hist <- last 3 pre-conv rows of (old hist ++ this call's rows); src/kernels.rs:173-190. */
void or_hist_update(const uint16_t* big, int stride, int L, int C, uint16_t* hist) {
    for (int c = 0; c < C; c++) {
        uint16_t v[3];
        for (int r = 0; r < 3; r++) {
            int src = L - 3 + r;
            v[r] = src >= 0 ? big[(int64_t)src * stride + c] : hist[(int64_t)(src + 3) * C + c];
        }
        for (int r = 0; r < 3; r++) hist[(int64_t)r * C + c] = v[r];
    }
}

/* ---- gated delta rule, sequential (src/kernels.rs:257-302) -------------------------------- */

/* qkv [L][2*H*DK + H*DV] f32 (conv output); a = big[t*stride + a_off + h], b at b_off (f16);
 * negA[H], dtb[H]; state [H][DK][DV] f32 (loaded when load_state, always written back);
 * o [L][H*DV] f32.  Per token: qn = q rsqrt(|q|^2 + 1e-6)/sqrt(DK), kn = k rsqrt(|k|^2 + 1e-6),
 * beta = sigmoid(b), g = negA * softplus(a + dtb) (softplus(x) = x for x > 20),
 * S *= e^g; delta = (v - S^T kn) beta; S += kn delta^T; o = S^T qn. */
void or_gdn(const float* qkv, const uint16_t* big, int stride, int a_off, int b_off, const float* negA,
            const float* dtb, int L, int H, int DK, int DV, float* state, int load_state, float* o) {
    int C = 2 * H * DK + H * DV;
#pragma omp parallel for schedule(static)
    for (int h = 0; h < H; h++) {
        float* S = state + (int64_t)h * DK * DV;
        if (!load_state) memset(S, 0, sizeof(float) * (size_t)DK * DV);
        float* qn = (float*)malloc(sizeof(float) * DK);
        float* kn = (float*)malloc(sizeof(float) * DK);
        float qs = 1.0f / sqrtf((float)DK);
        for (int t = 0; t < L; t++) {
            const float* q = qkv + (int64_t)t * C + h * DK;
            const float* k = qkv + (int64_t)t * C + H * DK + h * DK;
            const float* v = qkv + (int64_t)t * C + 2 * H * DK + h * DV;
            float sq = 0.0f, sk = 0.0f;
            for (int i = 0; i < DK; i++) {
                sq += q[i] * q[i];
                sk += k[i] * k[i];
            }
            float rq = 1.0f / sqrtf(sq + 1e-6f), rk = 1.0f / sqrtf(sk + 1e-6f);
            for (int i = 0; i < DK; i++) {
                qn[i] = q[i] * rq * qs;
                kn[i] = k[i] * rk;
            }
            float a = or_h2f(big[(int64_t)t * stride + a_off + h]);
            float b = or_h2f(big[(int64_t)t * stride + b_off + h]);
            float beta = 1.0f / (1.0f + expf(-b));
            float xx = a + dtb[h];
            float sp = xx > 20.0f ? xx : logf(1.0f + expf(xx));
            float decay = expf(negA[h] * sp);
            for (int c = 0; c < DV; c++) {
                float kv = 0.0f;
                for (int i = 0; i < DK; i++) {
                    S[i * DV + c] *= decay;
                    kv += S[i * DV + c] * kn[i];
                }
                float delta = (v[c] - kv) * beta;
                float oc = 0.0f;
                for (int i = 0; i < DK; i++) {
                    S[i * DV + c] += kn[i] * delta;
                    oc += S[i * DV + c] * qn[i];
                }
                o[(int64_t)t * H * DV + h * DV + c] = oc;
            }
        }
        free(qn);
        free(kn);
    }
}

/* ---- gated RMSNorm (src/kernels.rs:377-396) ---------------------------------------------- */

/* out[t, h*DV + c] = f16(w[c] * o * rsqrt(mean_c(o^2) + 1e-6) * silu(z)),
 * z = big[t*stride + z_off + h*DV + c]. */
void or_gnorm(const float* o, const uint16_t* big, int stride, int z_off, const float* w, int L, int H,
              int DV, uint16_t* out) {
    for (int t = 0; t < L; t++)
        for (int h = 0; h < H; h++) {
            int64_t b = (int64_t)t * H * DV + h * DV;
            float ss = 0.0f;
            for (int c = 0; c < DV; c++) ss += o[b + c] * o[b + c];
            float inv = 1.0f / sqrtf(ss / (float)DV + 1e-6f);
            for (int c = 0; c < DV; c++) {
                float z = or_h2f(big[(int64_t)t * stride + z_off + h * DV + c]);
                out[b + c] = or_f2h(w[c] * o[b + c] * inv * z / (1.0f + expf(-z)));
            }
        }
}

/* ---- RoPE table (src/engine.rs:259-267) -------------------------------------------------- */

/* table[t][rd/2][2] = (cos, sin) of t / theta^(2i/rd), angle in f64, stored f32. */
void or_rope_table(int ctx, int rd, double theta, float* table) {
    for (int t = 0; t < ctx; t++)
        for (int i = 0; i < rd / 2; i++) {
            double a = (double)t / pow(theta, (double)(2 * i) / (double)rd);
            table[(int64_t)t * rd + 2 * i] = (float)cos(a);
            table[(int64_t)t * rd + 2 * i + 1] = (float)sin(a);
        }
}

/* ---- q/k RMSNorm + partial rotate-half RoPE, K/V cache write (src/kernels.rs:400-448) ----- */

/* big [L][stride] f16 with q heads interleaved with their gates ([q | gate] per head, 2*HD
 * each), K at k_off = 2*HQ*HD, V at v_off = 2*HQ*HD + HK*HD.  Writes Qo [HQ][L][HD] f16 and rows
 * P..P+L-1 of Kc, Vc [HK][LT][HD] f16. */
void or_qk_prep(const uint16_t* big, int stride, const float* qw, const float* kw, const float* rope,
                int L, int P, int LT, int HQ, int HK, int HD, int RD, uint16_t* Qo, uint16_t* Kc, uint16_t* Vc) {
    int k_off = 2 * HQ * HD, v_off = 2 * HQ * HD + HK * HD, rd2 = RD / 2;
    float* n = (float*)malloc(sizeof(float) * HD);
    for (int t = 0; t < L; t++) {
        int pos = P + t;
        for (int s = 0; s < HQ + HK; s++) {
            int isq = s < HQ;
            if (!isq) {
                int kh = s - HQ;
                for (int d = 0; d < HD; d++)
                    Vc[((int64_t)kh * LT + pos) * HD + d] = big[(int64_t)t * stride + v_off + kh * HD + d];
            }
            const uint16_t* src = big + (int64_t)t * stride + (isq ? s * 2 * HD : k_off + (s - HQ) * HD);
            float tot = 0.0f;
            for (int d = 0; d < HD; d++) {
                float v = or_h2f(src[d]);
                tot += v * v;
            }
            float inv = 1.0f / sqrtf(tot / (float)HD + 1e-6f);
            const float* w = isq ? qw : kw;
            for (int d = 0; d < HD; d++) n[d] = or_h2f(src[d]) * inv * w[d];
            for (int d = 0; d < HD; d++) {
                float r = n[d];
                if (d < RD) {
                    int i = d % rd2;
                    float c = rope[((int64_t)pos * rd2 + i) * 2], sn = rope[((int64_t)pos * rd2 + i) * 2 + 1];
                    r = d < rd2 ? n[d] * c - n[d + rd2] * sn : n[d] * c + n[d - rd2] * sn;
                }
                if (isq) Qo[((int64_t)s * L + t) * HD + d] = or_f2h(r);
                else Kc[((int64_t)(s - HQ) * LT + pos) * HD + d] = or_f2h(r);
            }
        }
    }
    free(n);
}

/* ---- causal GQA attention with sigmoid gate (src/kernels.rs:453-541) ---------------------- */

/* Query t (absolute position P + t) of head h attends keys 0..P+t of kv head h / (HQ/HK).
 * q is pre-scaled by 1/sqrt(HD) and rounded to f16; scores in f32; softmax in f64 (the
 * reference's online softmax is the same quantity); out = f16(sum p v / sum p * sigmoid(gate)),
 * gate = big[t*stride + h*2*HD + HD + d]. */
void or_attn(const uint16_t* Qo, const uint16_t* Kc, const uint16_t* Vc, const uint16_t* big, int stride,
             int L, int P, int LT, int HQ, int HK, int HD, uint16_t* out) {
    float scale = (float)(1.0 / sqrt((double)HD));
    int gqa = HQ / HK;
#pragma omp parallel
    {
        float* q = (float*)malloc(sizeof(float) * HD);
        double* p = (double*)malloc(sizeof(double) * (size_t)(P + L));
        double* acc = (double*)malloc(sizeof(double) * HD);
#pragma omp for collapse(2) schedule(dynamic)
        for (int h = 0; h < HQ; h++)
            for (int t = 0; t < L; t++) {
                int kh = h / gqa, nk = P + t + 1;
                for (int d = 0; d < HD; d++) q[d] = rnd16(or_h2f(Qo[((int64_t)h * L + t) * HD + d]) * scale);
                double mx = -1e300;
                for (int j = 0; j < nk; j++) {
                    const uint16_t* k = Kc + ((int64_t)kh * LT + j) * HD;
                    float s = 0.0f;
                    for (int d = 0; d < HD; d++) s += q[d] * or_h2f(k[d]);
                    p[j] = s;
                    if (s > mx) mx = s;
                }
                double l = 0.0;
                for (int j = 0; j < nk; j++) {
                    p[j] = exp(p[j] - mx);
                    l += p[j];
                }
                for (int d = 0; d < HD; d++) acc[d] = 0.0;
                for (int j = 0; j < nk; j++) {
                    const uint16_t* v = Vc + ((int64_t)kh * LT + j) * HD;
                    for (int d = 0; d < HD; d++) acc[d] += p[j] * or_h2f(v[d]);
                }
                for (int d = 0; d < HD; d++) {
                    float g = or_h2f(big[(int64_t)t * stride + h * 2 * HD + HD + d]);
                    out[(int64_t)t * HQ * HD + h * HD + d] = or_f2h((float)(acc[d] / l) / (1.0f + expf(-g)));
                }
            }
        free(q);
        free(p);
        free(acc);
    }
}

/* ---- unrotate: in-place FWHT, Sylvester order, unnormalized (src/engine.rs:714-727) -------- */

void or_fwht(float* x, int n) {
    for (int h = 1; h < n; h *= 2)
        for (int i = 0; i < n; i += 2 * h)
            for (int j = i; j < i + h; j++) {
                float a = x[j], b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
}

int or_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
