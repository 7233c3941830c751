// Full-attention sublayer on gfx950: q/k RMSNorm + partial rotate-half RoPE with the K/V cache
// write (reference: src/kernels.rs:400-448), and causal GQA attention with a sigmoid output gate
// (reference: src/kernels.rs:453-541).
//
// Attention: a workgroup takes 16 queries of one q head and walks the keys in tiles of 64: the
// K tile is staged in LDS as f16, scores are f32, the softmax is online (running max and sum per
// query), and each thread accumulates one head dimension for the 16 queries.  When the query
// blocks alone cannot fill the GPU (the short question suffix over a long cached prefix), the
// key range is split over workgroups and a combine kernel merges the partial (max, sum, acc).
// As in the reference, q is pre-scaled by 1/sqrt(hd) and rounded to f16 before the dot products.
#include <cmath>

#include "common.h"

namespace sd {
namespace {

constexpr int BQ = 16;  // queries per workgroup
constexpr int KT = 64;  // keys per tile

template <int HD>
__global__ __launch_bounds__(HD) void k_qk_prep(const f16* __restrict__ big, AttnShape s, const float* __restrict__ qw,
                                                const float* __restrict__ kw, const float* __restrict__ rope, int L,
                                                const uint32_t* __restrict__ lu, f16* __restrict__ Q,
                                                f16* __restrict__ Kc, f16* __restrict__ Vc) {
    __shared__ float red[HD / 64];
    __shared__ float nv[HD];
    const int t = blockIdx.x, slot = blockIdx.y, d = threadIdx.x;
    const int pos = (int)lu[1] + t;
    const bool isq = slot < s.HQ;
    const int k_off = 2 * s.HQ * HD, v_off = k_off + s.HK * HD;
    const f16* row = big + (size_t)t * s.stride;
    if (!isq) {
        const int kh = slot - s.HQ;
        Vc[((size_t)kh * s.ctx + pos) * HD + d] = row[v_off + kh * HD + d];
    }
    const float v = (float)row[isq ? slot * 2 * HD + d : k_off + (slot - s.HQ) * HD + d];
    float ss = v * v;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if ((d & 63) == 0) red[d >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < HD / 64; i++) tot += red[i];
    const float n = v * (1.0f / sqrtf(tot / (float)HD + 1e-6f)) * (isq ? qw[d] : kw[d]);
    nv[d] = n;
    __syncthreads();
    float r = n;
    const int rd2 = s.RD / 2;
    if (d < s.RD) {
        const int i = d % rd2;
        const float c = rope[((size_t)pos * rd2 + i) * 2], sn = rope[((size_t)pos * rd2 + i) * 2 + 1];
        r = d < rd2 ? n * c - nv[d + rd2] * sn : n * c + nv[d - rd2] * sn;
    }
    if (isq) Q[((size_t)slot * L + t) * HD + d] = (f16)r;
    else Kc[((size_t)(slot - s.HQ) * s.ctx + pos) * HD + d] = (f16)r;
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn(const f16* __restrict__ Q, const f16* __restrict__ Kc,
                                              const f16* __restrict__ Vc, const f16* __restrict__ big, AttnShape s,
                                              int L, const uint32_t* __restrict__ lu, f16* __restrict__ out,
                                              float* __restrict__ pacc, float* __restrict__ pml, int ks) {
    static_assert(HD == 256, "attention is written for 256-wide heads (one thread per dimension)");
    constexpr int QP = HD + 4;  // padded f32 row
    constexpr int KP = HD + 8;  // padded f16 row
    __shared__ __attribute__((aligned(16))) float Qs[BQ * QP];
    __shared__ __attribute__((aligned(16))) f16 Ks[KT * KP];
    __shared__ float Ps[BQ][KT + 1];
    __shared__ float alpha_s[BQ];
    const int tid = threadIdx.x;
    const int P = (int)lu[1];
    const int t0 = blockIdx.x * BQ, h = blockIdx.y, z = blockIdx.z;
    const int kh = h / (s.HQ / s.HK);
    const int nq = min(BQ, L - t0);
    const int nkeys = P + t0 + nq;  // keys 0 .. P + t0 + nq - 1 can be attended
    const int span = ((nkeys + ks - 1) / ks + KT - 1) / KT * KT;
    const int kbeg = z * span, kend = min(nkeys, kbeg + span);
    const float scale = 1.0f / sqrtf((float)HD);

    for (int e = tid; e < BQ * HD; e += 256) {
        const int i = e / HD, d = e % HD;
        float q = 0.f;
        if (i < nq) q = (float)(f16)((float)Q[((size_t)h * L + t0 + i) * HD + d] * scale);
        Qs[i * QP + d] = q;
    }
    // score lanes: query qi, keys kj .. kj + 3 of the tile
    const int qi = tid >> 4, kj = (tid & 15) * 4;
    float m_run = -INFINITY, l_run = 0.f;  // valid in the 16 lanes owning query qi
    float acc[BQ];
#pragma unroll
    for (int i = 0; i < BQ; i++) acc[i] = 0.f;
    const f16* Kbase = Kc + (size_t)kh * s.ctx * HD;
    const f16* Vbase = Vc + (size_t)kh * s.ctx * HD;

    for (int j0 = kbeg; j0 < kend; j0 += KT) {
        __syncthreads();  // previous tile's Ks / Ps reads are done (and Qs is written)
        for (int e = tid; e < KT * HD / 8; e += 256) {
            const int j = e / (HD / 8), c8 = e % (HD / 8);
            f16x8 v = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
            if (j0 + j < kend) v = *reinterpret_cast<const f16x8*>(Kbase + (size_t)(j0 + j) * HD + c8 * 8);
            *reinterpret_cast<f16x8*>(&Ks[j * KP + c8 * 8]) = v;
        }
        __syncthreads();
        float sc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int d = 0; d < HD; d += 8) {
            const float4 qa = *reinterpret_cast<const float4*>(&Qs[qi * QP + d]);
            const float4 qb = *reinterpret_cast<const float4*>(&Qs[qi * QP + d + 4]);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const f16x8 k8 = *reinterpret_cast<const f16x8*>(&Ks[(kj + r) * KP + d]);
                sc[r] += qa.x * (float)k8[0] + qa.y * (float)k8[1] + qa.z * (float)k8[2] + qa.w * (float)k8[3] +
                         qb.x * (float)k8[4] + qb.y * (float)k8[5] + qb.z * (float)k8[6] + qb.w * (float)k8[7];
            }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int j = j0 + kj + r;
            if (!(j < kend && j <= P + t0 + qi && qi < nq)) sc[r] = -INFINITY;
            tmax = fmaxf(tmax, sc[r]);
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, o));
        const float m_new = fmaxf(m_run, tmax);
        float psum = 0.f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float p = sc[r] == -INFINITY ? 0.f : expf(sc[r] - m_new);
            Ps[qi][kj + r] = p;
            psum += p;
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) psum += __shfl_xor(psum, o);
        const float al = m_run == -INFINITY ? 0.f : expf(m_run - m_new);
        l_run = l_run * al + psum;
        m_run = m_new;
        if ((tid & 15) == 0) alpha_s[qi] = al;
        __syncthreads();
        const int d = tid;
#pragma unroll
        for (int i = 0; i < BQ; i++) acc[i] *= alpha_s[i];
        const int jn = min(KT, kend - j0);
        for (int jj = 0; jj < jn; jj++) {
            const float v = (float)Vbase[(size_t)(j0 + jj) * HD + d];
#pragma unroll
            for (int i = 0; i < BQ; i++) acc[i] += Ps[i][jj] * v;
        }
    }
    // per-query (m, l) to LDS so that the dimension threads can read them
    __shared__ float m_s[BQ], l_s[BQ];
    if ((tid & 15) == 0) {
        m_s[qi] = m_run;
        l_s[qi] = l_run;
    }
    __syncthreads();
    const int d = tid;
    if (ks == 1) {
        for (int i = 0; i < nq; i++) {
            const int t = t0 + i;
            const float g = (float)big[(size_t)t * s.stride + h * 2 * HD + HD + d];
            out[(size_t)t * s.HQ * HD + h * HD + d] = (f16)(acc[i] / l_s[i] / (1.0f + expf(-g)));
        }
    } else {
        for (int i = 0; i < nq; i++) {
            const size_t r = ((size_t)z * L + t0 + i) * s.HQ + h;
            pacc[r * HD + d] = acc[i];
            if (d == 0) {
                pml[r * 2] = m_s[i];
                pml[r * 2 + 1] = l_s[i];
            }
        }
    }
}

template <int HD>
__global__ __launch_bounds__(HD) void k_attn_combine(const float* __restrict__ pacc, const float* __restrict__ pml,
                                                     const f16* __restrict__ big, AttnShape s, int L, int ks,
                                                     f16* __restrict__ out) {
    const int t = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
    float m = -INFINITY;
    for (int z = 0; z < ks; z++) {
        const size_t r = ((size_t)z * L + t) * s.HQ + h;
        if (pml[r * 2 + 1] > 0.f) m = fmaxf(m, pml[r * 2]);
    }
    float l = 0.f, a = 0.f;
    for (int z = 0; z < ks; z++) {
        const size_t r = ((size_t)z * L + t) * s.HQ + h;
        const float lz = pml[r * 2 + 1];
        if (lz > 0.f) {
            const float f = expf(pml[r * 2] - m);
            l += lz * f;
            a += pacc[r * HD + d] * f;
        }
    }
    const float g = (float)big[(size_t)t * s.stride + h * 2 * HD + HD + d];
    out[(size_t)t * s.HQ * HD + h * HD + d] = (f16)(a / l / (1.0f + expf(-g)));
}

}  // namespace

void qk_prep(const f16* big, const AttnShape& s, const float* qw, const float* kw, const float* rope, int L,
             const uint32_t* lu, f16* Q, f16* Kc, f16* Vc, hipStream_t st) {
    SD_CHECK(s.HD == 256, "attention: only head_dim 256 is supported");
    SD_CHECK(s.RD % 2 == 0 && s.RD <= s.HD, "attention: bad rotary_dim");
    hipLaunchKernelGGL(k_qk_prep<256>, dim3(L, s.HQ + s.HK), dim3(256), 0, st, big, s, qw, kw, rope, L, lu, Q, Kc, Vc);
    launched("qk_prep");
}

// Workspace (floats) the key-split path needs for up to `rows` query rows.
size_t attn_ws_floats(int rows, const AttnShape& s) { return (size_t)8 * rows * s.HQ * (s.HD + 2); }

void attention_split(const f16* Q, const f16* Kc, const f16* Vc, const f16* big, const AttnShape& s, int L,
                     const uint32_t* lu, int ks, float* ws, f16* out, hipStream_t st) {
    SD_CHECK(s.HD == 256 && s.HQ % s.HK == 0, "attention: unsupported head shape");
    const int nb = (L + BQ - 1) / BQ;
    float* pacc = ws;
    float* pml = ws + (size_t)ks * L * s.HQ * s.HD;
    hipLaunchKernelGGL(k_attn<256>, dim3(nb, s.HQ, ks), dim3(256), 0, st, Q, Kc, Vc, big, s, L, lu, out, pacc, pml, ks);
    launched("attn");
    if (ks > 1) {
        hipLaunchKernelGGL(k_attn_combine<256>, dim3(L, s.HQ), dim3(256), 0, st, pacc, pml, big, s, L, ks, out);
        launched("attn_combine");
    }
}

}  // namespace sd
