// Gated delta net on gfx950: depthwise conv + SiLU, the chunked gated delta rule (chunk 64,
// fp32 accuracy), and the gated RMSNorm.  Reference kernels: src/kernels.rs:152-190 (conv,
// hist_update), 257-372 (the delta rule, sequential over tokens), 377-396 (gnorm).
//
// The reference runs the delta rule token by token: S <- e^g S; delta = (v - S^T kn) beta;
// S <- S + kn delta^T; o = S^T qn.  Here the same recurrence is evaluated per chunk of 64 tokens
// (the WY/UT form): with G the within-chunk cumulative log-decay,
//   A_ij = -beta_i (kn_i . kn_j) e^(G_i - G_j) (i > j),  T = (I - A)^-1,
//   W = T diag(beta e^G) Kn,  U = T diag(beta) V,  Qk_ij = (qn_i . kn_j) e^(G_i - G_j) (i >= j),
//   per chunk:  V' = U - W S;  o = (qn e^G) S + Qk V';  S <- e^(G_last) S + (Kn e^(G_last - G))^T V'.
// Every exponent above is <= 0, so nothing overflows for any decay.
//
// All matrix products run on v_mfma_f32_16x16x32_f16 with each fp32 operand split into
// hi = f16(x) and lo = f16(x - hi) and three MFMAs per product (hi.hi + hi.lo + lo.hi, f32
// accumulation): about 22 significant bits per operand, well inside the fp32 parity tolerance.
// Normalised q/k are scaled by 2^8 before the split (exact) so that small components stay in the
// f16 normal range.
//  * gdn_prep: one workgroup per (chunk, head), fully parallel: norms, decays, Kn Kn^T and Qn Kn^T,
//    T by a blocked inversion (16x16 diagonal blocks as (I+N)(I+N^2)(I+N^4)(I+N^8), then block
//    rows), W and U.  It writes the scan's A operands (W, qn e^G, Qk, (Kn e^(G_last-G))^T) already
//    split, in MFMA fragment order, so the scan reads each fragment with one 16-byte load per lane.
//    The workgroups also perform the reference's hist_update, each on a slice of the channels (the
//    conv already consumed the old history).
//  * gdn_scan: one workgroup per (head, 16 value columns), sequential over chunks; the state slice
//    lives in LDS (transposed, the B operand of every product); 4 waves carry the recurrence and 4
//    compute the output beside them.
#include "common.h"
#include "device.h"

namespace sd {
namespace {

constexpr int CH = 64;   // chunk length
constexpr int DVS = 16;  // value columns per scan workgroup (one MFMA column tile)
constexpr float QK_SCALE = 256.0f;

__device__ __forceinline__ float warp_sum8(float v) {  // sum over aligned groups of 8 lanes
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    return v;
}

// v = hi + lo with hi = f16(v) and lo = f16(v - hi), in pairs: one packed convert for two hi, the
// residual v - f32(hi) (exact in f32) by one v_fma_mix_f32 each (hi's half as an f16 operand, times
// -1, plus v), one packed convert for two lo: 12 VALU per 8 values instead of 32.
__device__ __forceinline__ void split8(const float* v, f16x8& hi, f16x8& lo) {
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        const f16x2 h = f16x2{(f16)v[e], (f16)v[e + 1]};
        float r0, r1;
#if defined(__HIP_DEVICE_COMPILE__)
        const uint32_t hb = __builtin_bit_cast(uint32_t, h);
        asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r0) : "v"(hb), "v"(v[e]));
        asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r1) : "v"(hb), "v"(v[e + 1]));
#else
        r0 = v[e] - (float)h[0];
        r1 = v[e + 1] - (float)h[1];
#endif
        hi[e] = h[0];
        hi[e + 1] = h[1];
        lo[e] = (f16)r0;
        lo[e + 1] = (f16)r1;
    }
}


// e^x on the hardware exp2 (v_exp_f32, about 1 ulp in f32); x <= 0 here, so the result is in (0, 1].
__device__ __forceinline__ float fexp(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
#else
    return expf(x);
#endif
}

__device__ __forceinline__ f32x4 mma3(const f16x8& ah, const f16x8& al, const f16x8& bh, const f16x8& bl, f32x4 acc) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, acc, 0, 0, 0);
    return acc;
}

// The same three products into three separate accumulators acc[0..2] (independent MFMA chains).
__device__ __forceinline__ void mma3s(const f16x8& ah, const f16x8& al, const f16x8& bh, const f16x8& bl, f32x4* acc) {
    acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, acc[1], 0, 0, 0);
    acc[2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, acc[2], 0, 0, 0);
}

// A-operand fragment store: matrix with KS k-steps of 32, layout [row tile][k step][hi|lo][lane][8].
__device__ __forceinline__ void put_frag(f16* base, int KS, int rt, int s, int lane, const float* v8) {
    f16x8 hi, lo;
    split8(v8, hi, lo);
    f16* p = base + ((size_t)((rt * KS + s) * 2) * 64 + lane) * 8;
    *reinterpret_cast<f16x8*>(p) = hi;
    *reinterpret_cast<f16x8*>(p + 64 * 8) = lo;
}


// The prefix snapshot's arena image whose GDN states and conv histories a forward continues from,
// read from the per-forward lu block (the device address at its byte 32; null when there is no lu
// or the prefix is the live arena's), so one captured plan serves every snapshot and the snapshot is
// read in place instead of being copied into the live arena first.
__device__ __forceinline__ const uint8_t* lu_prefix(const uint32_t* lu) {
    return lu ? *reinterpret_cast<const uint8_t* const*>(lu + 8) : nullptr;
}

// qkvc[t, c] = silu(sum_j w[c][j] x[t + j - 3, c]), rows before 0 from hist (src/kernels.rs:152-170).
// With several sequences, row t is index i of the sequence starting at row s0.
__global__ __launch_bounds__(256) void k_conv(const f16* __restrict__ big, int stride, int L, int C,
                                              const float* __restrict__ w, const f16* __restrict__ hist_live,
                                              float* __restrict__ out, const uint32_t* __restrict__ rowt, int R,
                                              const uint32_t* __restrict__ lu, size_t hist_off) {
    const uint8_t* pre = lu_prefix(lu);
    const f16* __restrict__ hist = pre ? reinterpret_cast<const f16*>(pre + hist_off) : hist_live;
    // 4 consecutive channels per thread (C % 4 == 0, checked by the launcher): 8-byte row loads,
    // 16-byte weight loads and stores; R consecutive rows per workgroup, so the weights are read
    // once per R rows and the rows a window shares come from L1
    const int c = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (c >= C) return;
    float4 kk[4];
#pragma unroll
    for (int u = 0; u < 4; u++) kk[u] = *reinterpret_cast<const float4*>(w + 4 * (c + u));
    const int tend = min(L, (int)(blockIdx.y + 1) * R);
    for (int t = blockIdx.y * R; t < tend; t++) {
        const int i = rowt ? (int)(rowt[t] & 0xFFFFu) : t;
        const int s0 = rowt ? (int)(rowt[t] >> 16) : 0;
        f16x4 xs[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int tt = i + j - 3;
            xs[j] = tt >= 0 ? *reinterpret_cast<const f16x4*>(big + (size_t)(s0 + tt) * stride + c)
                            : *reinterpret_cast<const f16x4*>(hist + (size_t)(tt + 3) * C + c);
        }
        float r[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float kj[4] = {kk[u].x, kk[u].y, kk[u].z, kk[u].w};
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < 4; j++) s += kj[j] * (float)xs[j][u];
            r[u] = s / (1.0f + expf(-s));
        }
        *reinterpret_cast<float4*>(out + (size_t)t * C + c) = float4{r[0], r[1], r[2], r[3]};
    }
}

// Workspace slot sizes (halves / floats) per (chunk, head).
constexpr size_t WF_H = 4 * 4 * 2 * 64 * 8;   // W: 4 row tiles x 4 k steps
constexpr size_t QGF_H = WF_H;                // qn e^G
constexpr size_t QKF_H = 4 * 2 * 2 * 64 * 8;  // Qk: 4 row tiles x 2 k steps
constexpr size_t KGF_H = 8 * 2 * 2 * 64 * 8;  // KgT: 8 row tiles x 2 k steps
constexpr size_t U_F = 64 * 128;              // U, fp32 [token][value column]

constexpr int PREP_T = 512;  // k_gdn_prep threads: 8 waves

// Two workgroups per (chunk, head), by role (blockIdx.z): role 0 builds T = (I - A)^-1 and from it
// W and U; role 1 the fragments that need no T (Qk, qn e^G, (Kn e^(G_last - G))^T), so the grid
// fills twice the CUs and the critical path is role 0 alone.  Two thread views
// of the chunk's rows:
//  - row view, thread (i, p) = (tid / 8, tid % 8): columns 16p..16p+15 of q and k in row i, for the
//    norms, the Q/K rows in LDS (the K Kn^T and Qn Kn^T operands) and the qn e^G fragments;
//  - column view, wave w, lane (n, g) = (lane % 16, lane / 16): column 16w + n of k and v at tokens
//    32s + 8g + u (s < 2, u < 8), loaded straight from global memory in that order, which is both an
//    MFMA B fragment over tokens (W = T diag(beta e^G) Kn and U = T diag(beta) V, column tile w) and
//    the scan's (Kn e^(G_last - G))^T A fragment (row tile w): no transpose passes through LDS.
// CONV: q, k and v are the causal conv + SiLU of big's rows, computed here (the reference's conv,
// src/kernels.rs:152-170: rows before a sequence's start from the history, the prefix snapshot's when
// lu names one); otherwise they are read from qkvc.
template <bool CONV>
// Kernel arguments: the pointers and ints first, the structs last (the first 16 dwords are preloaded
// into SGPRs, up to the first struct; the prologue needs the tables and big before anything else).
__global__ __attribute__((amdgpu_flat_work_group_size(PREP_T, PREP_T), amdgpu_waves_per_eu(4))) void k_gdn_prep(const uint32_t* __restrict__ chunkt, const uint32_t* __restrict__ lu,
                                                  const f16* __restrict__ big, const float* __restrict__ qkvc,
                                                  const float* __restrict__ negA, const float* __restrict__ dtb, int L,
                                                  GdnShape sh, GdnWs ws, ConvIn cv) {
    constexpr int DK = 128, DV = 128;
    constexpr int RP = DK + 8;  // f16 row pitch of the Q/K row tiles
    constexpr int FP = CH + 4;  // fp32 pitch of T and of the Qk staging
    constexpr int WP = DK + 4;  // fp32 pitch of the W staging
    // LDS regions: R1 = K rows (hi, lo), later W staging (fp32); R2 = Q rows (hi, lo), later Qk
    // staging (fp32); before both, the conv output (fp32 [token][XP], over R1 and R2); T; the blocks
    // of the inversion; per-token vectors.
    constexpr size_t R1B = 2 * CH * RP * 2 > CH * WP * 4 ? 2 * CH * RP * 2 : CH * WP * 4;
    constexpr int XP = 2 * 128 + 4;  // fp32 pitch of the conv output: two 128-channel matrices
    static_assert((size_t)CH * XP * 4 <= R1B + 2 * CH * RP * 2, "the conv output fits R1 and R2");
    __shared__ __attribute__((aligned(16))) uint8_t RR[R1B + 2 * CH * RP * 2];
    uint8_t* const R1 = RR;
    uint8_t* const R2 = RR + R1B;
    // T (the T side's) lives in R2: the T side stores no Q rows there, and the q side, which does,
    // has no T (its Qk staging takes the same place).  99 KB of LDS would fit one workgroup per CU;
    // 81.8 KB fits two (with at most 128 VGPRs), so a long input's chunks run in half the rounds.
    static_assert((size_t)CH * FP * 4 <= (size_t)2 * CH * RP * 2, "T fits R2");
    float* const Ts = reinterpret_cast<float*>(R2);
    __shared__ float Xs[4][16][17];
    __shared__ float Nb[6][16][17];  // the off-diagonal 16 x 16 blocks of A, (p, r) at p (p - 1) / 2 + r
    __shared__ __attribute__((aligned(16))) float beta[CH], G[CH], eG[CH], eL[CH], rkv[CH];
    f16* Kh = reinterpret_cast<f16*>(R1);
    f16* Kl = Kh + CH * RP;
    f16* Qh = reinterpret_cast<f16*>(R2);
    f16* Ql = Qh + CH * RP;

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int fr = lane & 15, fg = lane >> 4;  // fragment row (column) / k group of this lane
    const int c = blockIdx.x, h = blockIdx.y, H = sh.H;
    const bool qside = blockIdx.z != 0;  // role 1
    // The lu fields and the chunk's entry in one batch of scalar loads, issued before any branch:
    // the pointers are selected first, with `big` standing in for a null table (values then unused).
    const uint32_t* lp = lu ? lu : reinterpret_cast<const uint32_t*>(big);
    const uint32_t* cp = chunkt ? chunkt + c : lp;
    const uint32_t lu_chunks = lp[4], ce = *cp, lu_tree = lp[6];
    const uint8_t* const lu_pre = *reinterpret_cast<const uint8_t* const*>(lp + 8);
    SGPR_BATCH("s"(lu_chunks), "s"(ce), "s"(lu_tree), "s"(lu_pre), "s"(H), "s"(sh.C), "s"(sh.stride), "s"(sh.a_off), "s"(sh.b_off),
               "s"(sh.z_off), "s"(ws.wf), "s"(ws.qgf), "s"(ws.qkf), "s"(ws.kgf), "s"(ws.u), "s"(ws.gl), "s"(cv.w),
               "s"(cv.hist), "s"(cv.rowt), "s"(cv.hist_off), "s"(negA), "s"(dtb));
    if (chunkt && c >= (int)lu_chunks) return;  // the grid is sized for the most chunks L can split into
    const int t0 = chunkt ? (int)(ce & 0xFFFFu) : c * CH;
    const int Lc = chunkt ? (int)(ce >> 16) : min(CH, L - t0);
    // negA[h] and dtb[h] as vector loads (a scalar load would be waited for at the first LDS barrier)
    const float na = __builtin_bit_cast(float, buf_b32(make_rsrc(negA, (uint32_t)H * 4u), (uint32_t)h * 4u, 0u));
    const float db = __builtin_bit_cast(float, buf_b32(make_rsrc(dtb, (uint32_t)H * 4u), (uint32_t)h * 4u, 0u));
    const int C = sh.C;
    const size_t slot = (size_t)c * H + h;
    f16* Wf = ws.wf + slot * WF_H;
    f16* Qgf = ws.qgf + slot * QGF_H;
    f16* Qkf = ws.qkf + slot * QKF_H;
    f16* Kgf = ws.kgf + slot * KGF_H;
    float* Uo = ws.u + slot * U_F;  // U: [token][value column]

    // Every global load of the kernel is issued here, before its first store: vector memory
    // operations retire in issue order, so a load issued after a store would wait for its ack.  The
    // loads are unconditional (rows past the chunk read its last row; their scales and v are zeroed),
    // so no branch makes the wave wait for one load before it issues the next.
    const int ri = tid >> 3, rp = tid & 7;
    f16 ga16, gb16;  // the gate inputs of row tid % 64 (used by wave 0)
    {
        const size_t gr = (size_t)(t0 + min(tid & (CH - 1), Lc - 1)) * sh.stride + h;
        ga16 = big[gr + sh.a_off];
        gb16 = big[gr + sh.b_off];
    }
    float qv[16], kv[16];
    float kT[2][8], vT[2][8];  // column view (v on the T side only)
    if constexpr (!CONV) {
        {
            const float* row = qkvc + (size_t)(t0 + min(ri, Lc - 1)) * C;
            // the T side has no use for q: its "q" rows re-read k (same lines, no extra traffic)
            const float* rq4 = row + (qside ? h * DK : sh.H * DK + h * DK) + rp * 16;
            float4 q4[4], k4[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                q4[e] = *reinterpret_cast<const float4*>(rq4 + 4 * e);
                k4[e] = *reinterpret_cast<const float4*>(row + sh.H * DK + h * DK + rp * 16 + 4 * e);
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                qv[4 * e] = q4[e].x, qv[4 * e + 1] = q4[e].y, qv[4 * e + 2] = q4[e].z, qv[4 * e + 3] = q4[e].w;
                kv[4 * e] = k4[e].x, kv[4 * e + 1] = k4[e].y, kv[4 * e + 2] = k4[e].z, kv[4 * e + 3] = k4[e].w;
            }
        }
        const float* ck = qkvc + sh.H * DK + h * DK + wv * 16 + fr;
        const float* cvp = qkvc + 2 * sh.H * DK + h * DV + wv * 16 + fr;
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const size_t jr = (size_t)(t0 + min(s * 32 + fg * 8 + u, Lc - 1)) * C;
                kT[s][u] = ck[jr];
                vT[s][u] = qside ? 0.f : cvp[jr];
            }
    } else {
        // conv view: wave w takes tokens 8w..8w+7, lane l 4 channels of matrix l / 32 (q side: q, k;
        // T side: k, v); the 11 rows a wave's tokens read are the same for all its lanes, so whether
        // a row comes from big or from the history is wave-uniform.  A sequence's rows before its
        // first come from the history, except for a branch of a tree forward (lu[6] = the state's
        // length, a sequence starting past row 0), whose rows before its first are the state's last
        // rows (and before the state's first, the cleared history).
        const int wvu = __builtin_amdgcn_readfirstlane(wv);
        const int mat = lane >> 5, c4 = (lane & 31) * 4;
        const int m0 = qside ? (mat == 0 ? h * DK : sh.H * DK + h * DK) : (mat == 0 ? sh.H * DK + h * DK : 2 * sh.H * DK + h * DV);
        const int cg = m0 + c4;
        float4 wk[4];  // taps of the 4 channels
#pragma unroll
        for (int u = 0; u < 4; u++) wk[u] = *reinterpret_cast<const float4*>(cv.w + 4 * (cg + u));
        // the start row of the chunk's sequence (row table: index in the sequence | start row << 16)
        const int s0 = (int)((cv.rowt ? cv.rowt[t0] : (uint32_t)t0) >> 16);
        const int i0 = t0 - s0;  // the chunk's first row in its sequence
        const int tS = lu ? (int)lu_tree : 0;
        const bool branch = tS > 0 && s0 > 0;
        const uint8_t* pre = lu ? lu_pre : nullptr;
        const f16* hsrc = pre ? reinterpret_cast<const f16*>(pre + cv.hist_off) : cv.hist;
        const Rsrc rb = make_rsrc(big, (uint32_t)(t0 + Lc) * (uint32_t)sh.stride * 2u);
        const Rsrc rh = make_rsrc(hsrc, 3u * (uint32_t)C * 2u);
        f16x4 xr[11];
#pragma unroll
        for (int m = 0; m < 11; m++) {
            const int ii = min(i0 + 8 * wvu - 3 + m, i0 + Lc - 1);  // row of the sequence (uniform)
            // big's row, or (negative) history row rr + 3
            const int rr = ii >= 0 ? s0 + ii : branch ? tS + ii : ii;
            const bool fromh = rr < 0;
            const Rsrc r = fromh ? rh : rb;
            const uint32_t so = fromh ? (uint32_t)((rr + 3) * C) * 2u : (uint32_t)rr * (uint32_t)sh.stride * 2u;
            xr[m] = __builtin_bit_cast(f16x4, buf_b64(r, (uint32_t)cg * 2u, so));
        }
        float* X = reinterpret_cast<float*>(RR);
#pragma unroll
        for (int t = 0; t < 8; t++) {
            float o4[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float kj[4] = {wk[u].x, wk[u].y, wk[u].z, wk[u].w};
                float a = 0.f;
#pragma unroll
                for (int j = 0; j < 4; j++) a += kj[j] * (float)xr[t + j][u];
                o4[u] = silu(a);
            }
            *reinterpret_cast<float4*>(&X[(8 * wvu + t) * XP + mat * 128 + c4]) = float4{o4[0], o4[1], o4[2], o4[3]};
        }
        lds_barrier();
        const int mq = 0, mk = qside ? 128 : 0, mv = 128;
#pragma unroll
        for (int e = 0; e < 16; e += 4) {
            const float4 q4 = *reinterpret_cast<const float4*>(&X[ri * XP + mq + rp * 16 + e]);
            const float4 k4 = *reinterpret_cast<const float4*>(&X[ri * XP + mk + rp * 16 + e]);
            qv[e] = q4.x, qv[e + 1] = q4.y, qv[e + 2] = q4.z, qv[e + 3] = q4.w;
            kv[e] = k4.x, kv[e + 1] = k4.y, kv[e + 2] = k4.z, kv[e + 3] = k4.w;
        }
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int j = s * 32 + fg * 8 + u;
                kT[s][u] = X[j * XP + mk + wv * 16 + fr];
                vT[s][u] = qside ? 0.f : X[j * XP + mv + wv * 16 + fr];
            }
        lds_barrier();  // the conv output is consumed: R1 and R2 take the K and Q rows
    }

    // ---- phase 0: gates (wave 0), normalised q/k rows
    if (tid < CH) {
        const int i = tid;
        float b = 0.f, gl = 0.f;
        if (i < Lc) {
            const float a = (float)ga16, bb = (float)gb16;
            b = 1.0f / (1.0f + expf(-bb));
            const float x = a + db;
            const float sp = x > 20.0f ? x : logf(1.0f + expf(x));
            gl = na * sp;
        }
        float sc = gl;  // inclusive prefix sum over the 64 lanes of wave 0
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float v = __shfl_up(sc, o);
            if (i >= o) sc += v;
        }
        const float glast = __shfl(sc, Lc - 1);
        beta[i] = b;
        G[i] = sc;
        eG[i] = expf(sc);
        eL[i] = expf(glast - sc);
    }
    float rq;  // row view: 1 / |q_i| / sqrt(dk) (0 past the chunk)
    {
        float sq = 0.f, sk = 0.f;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            sq += qv[e] * qv[e];
            sk += kv[e] * kv[e];
        }
        sq = warp_sum8(sq);
        sk = warp_sum8(sk);
        const bool rin = ri < Lc;
        rq = rin ? (1.0f / sqrtf(sq + 1e-6f)) * (1.0f / sqrtf((float)DK)) : 0.f;
        const float rk = rin ? 1.0f / sqrtf(sk + 1e-6f) : 0.f;
        if (rp == 0) rkv[ri] = rk;
#pragma unroll
        for (int e = 0; e < 16; e += 8) {
            float q8[8], k8[8];
#pragma unroll
            for (int u = 0; u < 8; u++) q8[u] = qv[e + u] * rq * QK_SCALE, k8[u] = kv[e + u] * rk * QK_SCALE;
            f16x8 hi, lo;
            if (qside) {
                split8(q8, hi, lo);
                *reinterpret_cast<f16x8*>(&Qh[ri * RP + rp * 16 + e]) = hi;
                *reinterpret_cast<f16x8*>(&Ql[ri * RP + rp * 16 + e]) = lo;
            }
            split8(k8, hi, lo);
            *reinterpret_cast<f16x8*>(&Kh[ri * RP + rp * 16 + e]) = hi;
            *reinterpret_cast<f16x8*>(&Kl[ri * RP + rp * 16 + e]) = lo;
        }
    }
    lds_barrier();
    // qn e^G as A fragments: (row tile ri/16, k step rp/2, lanes (ri%16) + 16g, g = 2 (rp%2) + gg)
    if (qside) {
        const float e = eG[ri] * rq;
#pragma unroll
        for (int gg = 0; gg < 2; gg++) {
            float v8[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v8[u] = qv[gg * 8 + u] * e;
            put_frag(Qgf, 4, ri >> 4, rp >> 1, (ri & 15) + 16 * (2 * (rp & 1) + gg), v8);
        }
    }
    // column view: (Kn e^(G_last - G))^T fragments (row tile w), and the B fragments of phase 3
    f16x8 kbh[2], kbl[2], vbh[2], vbl[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int j0 = s * 32 + fg * 8;
        const float4 r0 = *reinterpret_cast<const float4*>(&rkv[j0]), r1 = *reinterpret_cast<const float4*>(&rkv[j0 + 4]);
        const float4 l0 = *reinterpret_cast<const float4*>(&eL[j0]), l1 = *reinterpret_cast<const float4*>(&eL[j0 + 4]);
        const float rk8[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
        const float el8[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
        float g8[8], k8[8], v8[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float kn = kT[s][u] * rk8[u];
            g8[u] = kn * el8[u];
            k8[u] = kn * QK_SCALE;
            v8[u] = j0 + u < Lc ? vT[s][u] : 0.f;
        }
        if (qside) {
            put_frag(Kgf, 2, wv, s, lane, g8);
        } else {
            split8(k8, kbh[s], kbl[s]);
            split8(v8, vbh[s], vbl[s]);
        }
    }

    // ---- phase 1: Kn Kn^T (T side) or Qn Kn^T (q side); wave w computes row tile w % 4 x column
    // tiles 2 (w / 4), 2 (w / 4) + 1
    {
        const int wr = wv & 3, tc = 2 * (wv >> 2);
        f32x4 acc[2];
#pragma unroll
        for (int t = 0; t < 2; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        const f16* Ah = qside ? Qh : Kh;
        const f16* Al = qside ? Ql : Kl;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int ar = (wr * 16 + fr) * RP + s * 32 + fg * 8;
            const f16x8 ah = *reinterpret_cast<const f16x8*>(&Ah[ar]), al = *reinterpret_cast<const f16x8*>(&Al[ar]);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int br = ((tc + t) * 16 + fr) * RP + s * 32 + fg * 8;
                const f16x8 kbh2 = *reinterpret_cast<const f16x8*>(&Kh[br]), kbl2 = *reinterpret_cast<const f16x8*>(&Kl[br]);
                acc[t] = mma3(ah, al, kbh2, kbl2, acc[t]);
            }
        }
        // the decays and beta this lane needs, read once: rows wr*16 + fg*4 + r, columns (tc+t)*16 + fr
        float Gi[4], Bi[4], Gj[2];
#pragma unroll
        for (int r = 0; r < 4; r++) Gi[r] = G[wr * 16 + fg * 4 + r], Bi[r] = beta[wr * 16 + fg * 4 + r];
#pragma unroll
        for (int t = 0; t < 2; t++) Gj[t] = G[(tc + t) * 16 + fr];
        lds_barrier();  // Q rows are consumed: R2 becomes the Qk staging area
        float* Qs = reinterpret_cast<float*>(R2);
        float* dst = qside ? Qs : Ts;
        constexpr float UNS = 1.0f / (QK_SCALE * QK_SCALE);
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int i = wr * 16 + fg * 4 + r, j = (tc + t) * 16 + fr;
                const float a = acc[t][r] * UNS * fexp(Gi[r] - Gj[t]);  // masked below where i < j
                const float vq = i >= j ? a : 0.f;
                const float vt = i > j ? -Bi[r] * a : (i == j ? 1.f : 0.f);
                dst[i * FP + j] = qside ? vq : vt;
            }
        lds_barrier();
        if (qside) {
            // Qk as A fragments: 4 row tiles x 2 k steps x 64 lanes, one per thread
            const int ln = tid & 63, st = (tid >> 6) & 1, rt = tid >> 7;
            const float* src = &Qs[(rt * 16 + (ln & 15)) * FP + st * 32 + (ln >> 4) * 8];
            float v8[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v8[u] = src[u];
            put_frag(Qkf, 2, rt, st, ln, v8);
            return;
        }
    }

    // ---- phase 2: T = (I - A)^-1 in place (Ts holds I + A, A strictly lower), in 16 x 16 blocks.
    // Diagonal block b (wave b < 4): forward substitution, lane j < 16 holding column j of
    // T_bb = (I - A_bb)^-1 in registers: T[i][j] = delta_ij + sum_{k<i} A[i][k] T[k][j].
    // The off-diagonal blocks of A are copied aside first, since T_pq overwrites A_pq.
    {
        const int base = wv * 16;
        for (int e = tid; e < 6 * 256; e += PREP_T) {
            const int blk = e >> 8, a = (e >> 4) & 15, b = e & 15;
            const int p = blk == 0 ? 1 : (blk < 3 ? 2 : 3), r = blk - p * (p - 1) / 2;
            Nb[blk][a][b] = Ts[(16 * p + a) * FP + 16 * r + b];
        }
        if (wv < 4 && lane < 16) {
            // right-looking: once x[k] is final it is added into every later row's sum, so the 16
            // rows' sums run side by side (the terms of each still add in k order)
            float x[16];
#pragma unroll
            for (int i = 0; i < 16; i++) x[i] = i == lane ? 1.f : 0.f;
#pragma unroll
            for (int k = 0; k < 15; k++)
#pragma unroll
                for (int i = k + 1; i < 16; i++) x[i] += Ts[(base + i) * FP + base + k] * x[k];
#pragma unroll
            for (int i = 0; i < 16; i++) Ts[(base + i) * FP + base + lane] = x[i];
        }
        lds_barrier();
    }
    // Off-diagonal blocks: column block q by wave q < 4, block rows p = q+1..3 in order (no workgroup
    // barrier: a wave reads only the final diagonal blocks, the copied A blocks and its own column):
    // T_pq = T_pp X, X = sum_{r=q}^{p-1} A_pr T_rq, each 16 x 16 x 16 product as 4 f32 MFMAs
    // (v_mfma_f32_16x16x4_f32: lane l holds A[l % 16][k0 + l / 16], B[k0 + l / 16][l % 16] and
    // D[4 (l / 16) + r][l % 16]).  X passes through the wave's own LDS block to become an operand.
    {
        const int q = wv, lr = lane & 15, lg = lane >> 4;
        float(&Xw)[16][17] = Xs[wv & 3];
        for (int p = q + 1; p < 4; p++) {  // waves 4-7: no block rows
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
            for (int r = q; r < p; r++) {
                const int blk = p * (p - 1) / 2 + r;
#pragma unroll
                for (int k0 = 0; k0 < 16; k0 += 4)
                    x = __builtin_amdgcn_mfma_f32_16x16x4f32(Nb[blk][lr][k0 + lg], Ts[(16 * r + k0 + lg) * FP + 16 * q + lr],
                                                             x, 0, 0, 0);
            }
#pragma unroll
            for (int rr = 0; rr < 4; rr++) Xw[4 * lg + rr][lr] = x[rr];
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's writes land before its reads
            f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k0 = 0; k0 < 16; k0 += 4)
                y = __builtin_amdgcn_mfma_f32_16x16x4f32(Ts[(16 * p + lr) * FP + 16 * p + k0 + lg], Xw[k0 + lg][lr], y, 0, 0, 0);
#pragma unroll
            for (int rr = 0; rr < 4; rr++) Ts[(16 * p + 4 * lg + rr) * FP + 16 * q + lr] = y[rr];
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // X is read before the next p writes it
        }
        lds_barrier();
    }

    // ---- phase 3: W = T diag(beta e^G) Kn and U = T diag(beta) V, column tile w of each (wave w),
    // all 4 row tiles; the B fragments are this lane's column view
    {
        float bw[2][8], bu[2][8];  // beta e^G and beta at tokens 32s + 8g + u
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int j0 = s * 32 + fg * 8;
#pragma unroll
            for (int u = 0; u < 8; u++) bu[s][u] = beta[j0 + u], bw[s][u] = beta[j0 + u] * eG[j0 + u];
        }
        f32x4 aw[4], au[4];
#pragma unroll
        for (int rt = 0; rt < 4; rt++) {
            aw[rt] = au[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 2; s++) {
                const float* tp = &Ts[(rt * 16 + fr) * FP + s * 32 + fg * 8];
                const float4 t0v = *reinterpret_cast<const float4*>(tp), t1v = *reinterpret_cast<const float4*>(tp + 4);
                const float t8[8] = {t0v.x, t0v.y, t0v.z, t0v.w, t1v.x, t1v.y, t1v.z, t1v.w};
                float xw[8], xu[8];
#pragma unroll
                for (int u = 0; u < 8; u++) xw[u] = t8[u] * bw[s][u], xu[u] = t8[u] * bu[s][u];
                f16x8 ah, al;
                split8(xw, ah, al);
                aw[rt] = mma3(ah, al, kbh[s], kbl[s], aw[rt]);
                split8(xu, ah, al);
                au[rt] = mma3(ah, al, vbh[s], vbl[s], au[rt]);
            }
        }
        // U straight to global (row-major); W through LDS (R1: the K rows are consumed)
        float* Ws = reinterpret_cast<float*>(R1);
#pragma unroll
        for (int rt = 0; rt < 4; rt++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                Uo[(rt * 16 + fg * 4 + r) * DV + wv * 16 + fr] = au[rt][r];
                Ws[(rt * 16 + fg * 4 + r) * WP + wv * 16 + fr] = aw[rt][r] * (1.0f / QK_SCALE);
            }
        }
        lds_barrier();
#pragma unroll
        for (int q = 0; q < 1024 / PREP_T; q++) {
            const int slotf = tid + PREP_T * q;  // 4 row tiles x 4 k steps x 64 lanes
            const int ln = slotf & 63, st = (slotf >> 6) & 3, rt = slotf >> 8;
            const float* src = &Ws[(rt * 16 + (ln & 15)) * WP + st * 32 + (ln >> 4) * 8];
            float v8[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v8[u] = src[u];
            put_frag(Wf, 4, rt, st, ln, v8);
        }
    }
    if (tid == 0) ws.gl[slot] = eG[Lc - 1];
}

// Sum over the 16 lanes of this lane's DPP row, the same bits in every lane: partners by mirror,
// half mirror, then quad xor 2 and xor 1, so each lane adds the same pairs in the same grouping.
__device__ __forceinline__ float dpp_f(float x, int ctrl) {
    switch (ctrl) {  // the control is an immediate of the instruction
        case 0x140: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x140, 0xF, 0xF, false));
        case 0x141: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x141, 0xF, 0xF, false));
        case 0x4E: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false));
        default: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
    }
}
__device__ __forceinline__ float row_allsum16(float x) {
    x += dpp_f(x, 0x140);  // row_mirror: lane i and 15 - i
    x += dpp_f(x, 0x141);  // row_half_mirror: i and 7 - i within each half
    x += dpp_f(x, 0x4E);   // quad_perm [2,3,0,1]
    x += dpp_f(x, 0xB1);   // quad_perm [1,0,3,2]
    return x;
}

// The reference's own token-by-token delta rule (src/kernels.rs:280-297) for short inputs (the
// questions of an ask_all): the chunked form's fixed cost per 64-token chunk outweighs a few dozen
// sequential steps.  Per token t and head h: qn = q rsqrt(q.q + 1e-6) / sqrt(dk), kn = k rsqrt(k.k
// + 1e-6), beta = sigmoid(b), decay = exp(negA softplus(a + dt_bias)); per value column:
// S *= decay; delta = (v - S^T kn) beta; S += kn delta; o = S^T qn (evaluated as below, with both
// column sums taken from the previous state).
// Workgroup (head, 32 value columns, sequence), 8 waves: wave w owns columns 32 y + 4 w + l / 16 and
// lane l state rows 8 (l % 16) .. + 7, so every reduction over a column's 128 rows is one DPP row.  The
// state stays in registers.  The inputs of up to 64 tokens are staged in LDS by the whole
// workgroup with wide loads (their latency is paid once per block, not per token).
// CONV: q, k and v are the causal conv + SiLU of big's rows, computed here per block (the
// reference's conv, src/kernels.rs:152-170; a sequence's first rows read the prefix's history): q
// and k in a conv view (wave w takes the block's tokens 8w .. 8w + 7, lane l 4 channels of q or k,
// so whether a row comes from big or from the history is wave-uniform) into LDS, over the Q/K
// tiles; the 32 v columns one (token, 4 channels) per thread.  Otherwise they are read from qkvc.
// Every workgroup of a head computes the head's q/k conv: 8 waves halve each one's share of it
// (and of the norms), and a head takes 4 workgroups instead of 8.
// With CONV the history is only read: the caller updates no history in the same launch.
constexpr int RTB = 64;           // tokens per LDS block
constexpr int RT = 512, RC = 32;  // threads and value columns per workgroup
template <bool CONV>
__global__ __launch_bounds__(RT) void k_gdn_recur(const uint32_t* __restrict__ lu, const uint32_t* __restrict__ seqt,
                                                   float* __restrict__ state, const f16* __restrict__ big,
                                                   const float* __restrict__ qkvc, int L, int load_default,
                                                   size_t state_off, const float* __restrict__ negA,
                                                   const float* __restrict__ dtb, float* __restrict__ o,
                                                   const uint32_t* __restrict__ chunkt, f16* hist, size_t hist_off,
                                                   GdnShape sh, ConvIn cv) {
    constexpr int DK = 128, DV = 128;
    // Q and K tiles of a block; with CONV first the conv output of q and k, f32 [token][256]
    __shared__ __attribute__((aligned(16))) float4 QKs[2 * RTB * DK / 4];
    float4 (*const Qs)[DK / 4] = reinterpret_cast<float4 (*)[DK / 4]>(QKs);
    float4 (*const Ks)[DK / 4] = reinterpret_cast<float4 (*)[DK / 4]>(QKs + RTB * DK / 4);
    float* const X = reinterpret_cast<float*>(QKs);
    __shared__ __attribute__((aligned(16))) float Vs[RTB][RC];
    __shared__ float Os[RTB][RC];
    __shared__ float4 Tg[RTB];  // decay, beta and kn . qn of a token (one 16-byte read)
    __shared__ float4 Wt[64 + RC / 4][4];  // CONV: the taps of the q/k view's 64 lane groups, then the v view's 8
    __shared__ float Ss[DK][RC + 1];      // the state slice on its way into the token loop's registers
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int h = blockIdx.x, H = sh.H, q = blockIdx.z;
    // The lu fields and the sequence's row range in one batch of scalar loads, issued before any
    // branch (a load behind one waits for the loads the branch needs): the pointers are selected
    // first, with `state` standing in for a null table (values then unused).
    const uint32_t* lp = lu ? lu : reinterpret_cast<const uint32_t*>(state);
    const uint32_t* sp = seqt ? seqt + SD_MAX_SEQS + q : lp;
    const uint32_t lu_nseq = lp[5], lu_load = lp[3], rr = *sp;
    const uint8_t* const lu_pre = *reinterpret_cast<const uint8_t* const*>(lp + 8);
    SGPR_BATCH("s"(lu_nseq), "s"(lu_load), "s"(rr), "s"(lu_pre), "s"(sh.H), "s"(sh.C), "s"(sh.stride), "s"(sh.a_off),
               "s"(sh.b_off), "s"(negA), "s"(dtb), "s"(o), "s"(cv.w), "s"(cv.hist), "s"(cv.hist_off));
    if (seqt && q >= (int)lu_nseq) return;  // the grid is sized for the most sequences
    // lane l of a 16-lane row owns state rows 4l .. 4l + 3 and 64 + 4l .. 64 + 4l + 3: its q and k
    // values are then float4 l and 16 + l of a token's row, so the 16 lanes of each read cover 256
    // contiguous bytes (every LDS bank once)
    const int cb = blockIdx.y * RC, cl = wv * 4 + (lane >> 4), col = cb + cl, l4 = lane & 15;
    auto srow = [&](int i) { return (i < 4 ? 0 : 60) + 4 * l4 + i; };
    int t0 = 0, t1 = L;
    if (seqt) {  // the sequence's rows (the chunk table would be a second, dependent load)
        t0 = (int)(rr & 0xFFFFu);
        t1 = t0 + (int)(rr >> 16);
    }
    const bool load = lu ? lu_load != 0u : load_default != 0;
    const uint8_t* pre = lu ? lu_pre : nullptr;
    float* Sg = state + (size_t)h * DK * DV;  // the live state (written back by a single sequence)
    const float* S0 = (pre ? reinterpret_cast<const float*>(pre + state_off) : state) + (size_t)h * DK * DV;
    // Every global load below is unconditional (indices clamped, values zeroed after they arrive): a
    // load under a branch makes the wave wait for it before it issues the next.
    // The state slice (128 rows x 32 columns) in 16-byte loads, two per thread, through a buffer
    // resource (a flat load, the prefix or live pointer not being known to be global, would also
    // count as an LDS operation and hold up the first LDS barrier); it reaches the token loop's
    // register layout through LDS with the first block's inputs.  One 4-byte load per register
    // would be 4x the vector-memory instructions, which the workgroup's prologue is bound by.
    // (The 16 bytes are reinterpreted as a whole: a bit_cast of one element of the loaded vector
    // compiles to a 4-byte load of element 0 with this compiler.)
    float4 sl[2];
    {
        const Rsrc rs = make_rsrc(S0, (uint32_t)(DK * DV * 4));
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int e = tid + RT * j;
            sl[j] = __builtin_bit_cast(float4, buf_b128(rs, (uint32_t)(((e >> 3) * DV + cb + 4 * (e & 7)) * 4), 0u));
        }
    }
    float S[8];
    bool fresh = !load;  // the state starts at zero: applied at the first token, after the block's loads
    const int C = sh.C;
    // negA[h] and dtb[h] as vector loads: a scalar load would be waited for at the block's first LDS
    // barrier (s_waitcnt lgkmcnt(0)), and they are needed only after the block's inputs arrive
    // (wave 0 only: the gates are computed for tokens tid < 64)
    float na = 0.f, db = 0.f;
    if (__builtin_amdgcn_readfirstlane(wv) == 0) {
        na = __builtin_bit_cast(float, buf_b32(make_rsrc(negA, (uint32_t)H * 4u), (uint32_t)h * 4u, 0u));
        db = __builtin_bit_cast(float, buf_b32(make_rsrc(dtb, (uint32_t)H * 4u), (uint32_t)h * 4u, 0u));
    }
    const float qs = 1.0f / sqrtf((float)DK);
    // conv views: lane l of the q/k view takes channels cg .. cg + 3 (matrix l / 32); thread (tv, vq)
    // of the v view takes token tv of the block and channels vg .. vg + 3
    const int cmat = lane >> 5, c4 = (lane & 31) * 4;
    const int cg = (cmat == 0 ? h * DK : sh.H * DK + h * DK) + c4;
    const int vq = tid & 7, tv = tid >> 3;
    const int vg = 2 * sh.H * DK + h * DV + cb + 4 * vq;
    // CONV: the taps the views use (72 groups of 4 channels x 4 taps, 4.5 KB) are loaded once per
    // workgroup, one float4 per thread (threads past 287 re-read the last), and shared through LDS;
    // every lane loading its own 8 float4 was 64 KB of vector-memory traffic per workgroup
    float4 wk[4], wvt[4], tap = {};
    const f16* hsrc = nullptr;
    if constexpr (CONV) {
        const int g = min(tid >> 2, 64 + RC / 4 - 1), p = tid & 3;
        const int ch = g < 64 ? ((g >> 5) == 0 ? h * DK : sh.H * DK + h * DK) + (g & 31) * 4 + p
                              : 2 * sh.H * DK + h * DV + cb + 4 * (g - 64) + p;
        tap = *reinterpret_cast<const float4*>(cv.w + 4 * ch);
        hsrc = pre ? reinterpret_cast<const f16*>(pre + cv.hist_off) : cv.hist;
    }
    for (int tb = t0; tb < t1; tb += RTB) {
        const int nt = min(RTB, t1 - tb);
        if (tb != t0) lds_barrier();  // the previous block's LDS is consumed
        // q and k of a token: one DPP row of 16 lanes x 8 values, normalised on the way into LDS
        // (the sums over the row are one row_allsum16).  Every load of the block is issued before
        // the first is used.
        constexpr int NIT = RTB * 16 / RT;  // token passes: 32 tokens per pass of the workgroup
        constexpr int NV = RTB * RC / RT;   // v values per thread
        float4 qr[NIT][2], kr[NIT][2];
        float vr[NV];
        f16 ga = 0, gb = 0;  // the gate inputs of token tid (used for tid < nt; converted there, so that
                             // no wait for the loads follows them)
        if constexpr (CONV) {
            // rows of the block by sequence index (rows past the sequence read its last row; the
            // outputs they feed are never used); index < 0: the history
            const int wvu = __builtin_amdgcn_readfirstlane(wv);
            const int ib = tb - t0, ilast = t1 - t0 - 1;
            const Rsrc rb = make_rsrc(big, (uint32_t)t1 * (uint32_t)sh.stride * 2u);
            const Rsrc rh = make_rsrc(hsrc, 3u * (uint32_t)C * 2u);
            f16x4 xr[11];
#pragma unroll
            for (int m = 0; m < 11; m++) {
                const int ii = min(ib + 8 * wvu - 3 + m, ilast);
                const bool fromh = ii < 0;
                const uint32_t so = fromh ? (uint32_t)((ii + 3) * C) * 2u : (uint32_t)(t0 + ii) * (uint32_t)sh.stride * 2u;
                xr[m] = __builtin_bit_cast(f16x4, buf_b64(fromh ? rh : rb, (uint32_t)cg * 2u, so));
            }
            // the v view: each thread loads its own token's row, the threads of the block's first 3
            // tokens also the row 3 before (the history at a sequence start); the conv reads its 4 rows
            // from LDS (Vr, over Os, which only the token loop writes) after the barrier.  Global loads
            // (a flat one would also count as an LDS operation).
            typedef __attribute__((address_space(1))) const f16x4 gf16x4;
            f16x4 (*const Vr)[RC / 4] = reinterpret_cast<f16x4 (*)[RC / 4]>(&Os[0][0]);
            const f16x4 vown = *(gf16x4*)(big + (size_t)(t0 + min(ib + tv, ilast)) * sh.stride + vg);
            f16x4 vprev = {};
            if (tv < 3) {
                const int ii = min(ib + tv - 3, ilast);
                const f16* src = ii < 0 ? hsrc + (size_t)(ii + 3) * C + vg : big + (size_t)(t0 + ii) * sh.stride + vg;
                vprev = *(gf16x4*)src;
            }
            {  // the gate inputs of token tid (used for tid < nt <= 64; under a branch, the wave would
               // wait for them there)
                const size_t gr = (size_t)(tb + min(tid, nt - 1)) * sh.stride + h;
                ga = big[gr + sh.a_off];
                gb = big[gr + sh.b_off];
            }
            if (tb == t0) {  // the taps into LDS, then into the registers of both views
                if (tid < (64 + RC / 4) * 4) Wt[tid >> 2][tid & 3] = tap;
                lds_barrier();
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    wk[u] = Wt[lane][u];  // the q/k view's group of lane l is l
                    wvt[u] = Wt[64 + vq][u];
                }
            }
#pragma unroll
            for (int t = 0; t < 8; t++) {
                float o4[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float kj[4] = {wk[u].x, wk[u].y, wk[u].z, wk[u].w};
                    float a = 0.f;
#pragma unroll
                    for (int j = 0; j < 4; j++) a += kj[j] * (float)xr[t + j][u];
                    o4[u] = silu(a);
                }
                *reinterpret_cast<float4*>(&X[(8 * wvu + t) * 256 + cmat * 128 + c4]) = float4{o4[0], o4[1], o4[2], o4[3]};
            }
            Vr[tv + 3][vq] = vown;  // Vr row i: token i - 3 of the block
            if (tv < 3) Vr[tv][vq] = vprev;
            lds_barrier();
            {
                f16x4 vx[4];
#pragma unroll
                for (int j = 0; j < 4; j++) vx[j] = Vr[tv + j][vq];
                float o4[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float kj[4] = {wvt[u].x, wvt[u].y, wvt[u].z, wvt[u].w};
                    float a = 0.f;
#pragma unroll
                    for (int j = 0; j < 4; j++) a += kj[j] * (float)vx[j][u];
                    o4[u] = silu(a);
                }
                *reinterpret_cast<float4*>(&Vs[tv][4 * vq]) = float4{o4[0], o4[1], o4[2], o4[3]};
            }
#pragma unroll
            for (int it = 0; it < NIT; it++) {
                const int e = it * RT + tid, tt = e >> 4, j = e & 15;
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    qr[it][u] = *reinterpret_cast<const float4*>(&X[tt * 256 + 8 * j + 4 * u]);
                    kr[it][u] = *reinterpret_cast<const float4*>(&X[tt * 256 + 128 + 8 * j + 4 * u]);
                }
            }
            lds_barrier();  // X is read: the Q/K tiles overwrite it
        } else {
#pragma unroll
            for (int it = 0; it < NIT; it++) {
                const int e = it * RT + tid, tt = e >> 4, j = e & 15;
                const float* row = qkvc + (size_t)(tb + min(tt, nt - 1)) * C;  // tokens past the block: unused
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    qr[it][u] = *reinterpret_cast<const float4*>(row + h * DK + 8 * j + 4 * u);
                    kr[it][u] = *reinterpret_cast<const float4*>(row + sh.H * DK + h * DK + 8 * j + 4 * u);
                }
            }
#pragma unroll
            for (int it = 0; it < NV; it++) {
                const int e = it * RT + tid;
                vr[it] = qkvc[(size_t)(tb + min(e / RC, nt - 1)) * C + 2 * sh.H * DK + h * DV + cb + e % RC];
            }
            const size_t gr = (size_t)(tb + min(tid, nt - 1)) * sh.stride + h;
            ga = big[gr + sh.a_off];
            gb = big[gr + sh.b_off];
        }
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int e = it * RT + tid, tt = e >> 4, j = e & 15;
            float sq = 0.f, sk = 0.f, kq = 0.f;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const float4 q4 = qr[it][u], k4 = kr[it][u];
                sq += q4.x * q4.x + q4.y * q4.y + q4.z * q4.z + q4.w * q4.w;
                sk += k4.x * k4.x + k4.y * k4.y + k4.z * k4.z + k4.w * k4.w;
                kq += q4.x * k4.x + q4.y * k4.y + q4.z * k4.z + q4.w * k4.w;
            }
            sq = row_allsum16(sq);
            sk = row_allsum16(sk);
            kq = row_allsum16(kq);
            const float rq = 1.0f / sqrtf(sq + 1e-6f), rk = 1.0f / sqrtf(sk + 1e-6f);
            if (tt < nt) {
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const float4 q4 = qr[it][u], k4 = kr[it][u];
                    Qs[tt][2 * j + u] = float4{q4.x * rq * qs, q4.y * rq * qs, q4.z * rq * qs, q4.w * rq * qs};
                    Ks[tt][2 * j + u] = float4{k4.x * rk, k4.y * rk, k4.z * rk, k4.w * rk};
                }
                if (j == 0) Tg[tt].z = kq * rq * qs * rk;
            }
        }
        if constexpr (!CONV) {
#pragma unroll
            for (int it = 0; it < NV; it++) {
                const int e = it * RT + tid;
                if (e / RC < nt) Vs[e / RC][e % RC] = vr[it];
            }
        }
        if (tid < nt) {
            const float x = (float)ga + db;
            const float sp = x > 20.0f ? x : logf(1.0f + expf(x));
            Tg[tid].x = expf(na * sp);
            Tg[tid].y = 1.0f / (1.0f + expf(-(float)gb));
        }
        if (tb == t0) {  // the state slice: Ss[row][c] = S0[row][cb + c]
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int e = tid + RT * j, r = e >> 3, c = 4 * (e & 7);
#pragma unroll
                for (int k = 0; k < 4; k++) Ss[r][c + k] = k == 0 ? sl[j].x : k == 1 ? sl[j].y : k == 2 ? sl[j].z : sl[j].w;
            }
        }
        __syncthreads();
        if (tb == t0) {
#pragma unroll
            for (int i = 0; i < 8; i++) S[i] = Ss[srow(i)][cl];
        }
        if (fresh) {
#pragma unroll
            for (int i = 0; i < 8; i++) S[i] = 0.f;
            fresh = false;
        }
        // Both column sums come from the previous state, so they are independent:
        //   S_t = dc S + kn delta^T, delta = beta (v - dc S^T kn), o = S_t^T qn = dc S^T qn + (kn . qn) delta
        // A token's operands do not depend on the state: those of token tt + 1 are read from LDS
        // while token tt runs (the chain per token is then FMAs and DPP sums only).
        struct Tok {
            float4 qa, qb, ka, kb, gt;
            float v;
        };
        auto tok = [&](int tt) { return Tok{Qs[tt][l4], Qs[tt][16 + l4], Ks[tt][l4], Ks[tt][16 + l4], Tg[tt], Vs[tt][cl]}; };
        auto run = [&](const Tok& x, int tt) {
            const float qn[8] = {x.qa.x, x.qa.y, x.qa.z, x.qa.w, x.qb.x, x.qb.y, x.qb.z, x.qb.w};
            const float kn[8] = {x.ka.x, x.ka.y, x.ka.z, x.ka.w, x.kb.x, x.kb.y, x.kb.z, x.kb.w};
            const float dc = x.gt.x;
            float sk = 0.f, sq = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                sk += S[i] * kn[i];
                sq += S[i] * qn[i];
            }
            sk = row_allsum16(sk);
            sq = row_allsum16(sq);
            const float delta = (x.v - dc * sk) * x.gt.y;
            const float oc = dc * sq + x.gt.z * delta;
#pragma unroll
            for (int i = 0; i < 8; i++) S[i] = dc * S[i] + kn[i] * delta;
            if ((lane & 15) == 0) Os[tt][cl] = oc;
        };
        // two tokens per iteration, their operand sets alternating (no register copies)
        Tok ta = tok(0);
        int tt = 0;
        for (; tt + 1 < nt; tt += 2) {
            const Tok tb2 = tok(tt + 1);
            run(ta, tt);
            ta = tok(min(tt + 2, nt - 1));
            run(tb2, tt + 1);
        }
        if (tt < nt) run(ta, tt);
        // the block's outputs leave as whole 128-byte rows (32 columns of a token)
        __syncthreads();
#pragma unroll
        for (int it = 0; it < RTB * RC / RT; it++) {
            const int e = it * RT + tid, r = e / RC;
            if (r < nt) o[(size_t)(tb + r) * sh.H * DV + h * DV + cb + e % RC] = Os[r][e % RC];
        }
    }
    if (seqt) return;  // several sequences: their final states are not kept
#pragma unroll
    for (int i = 0; i < 8; i++) Sg[(size_t)srow(i) * DV + col] = S[i];
    // the reference's hist_update (src/kernels.rs:173-190), each workgroup on a slice of the channels:
    // the last 3 rows of (the prefix's history ++ this forward's rows) into the live history
    if (hist) {
        const f16* old = pre ? reinterpret_cast<const f16*>(pre + hist_off) : hist;
        const int nb = H * (DV / RC), per = (C + nb - 1) / nb, bi = blockIdx.y * H + h;
        const int lo = bi * per, hi = min(C, lo + per);
        for (int ch = lo + tid; ch < hi; ch += RT) {
            f16 hv[3];
#pragma unroll
            for (int r = 0; r < 3; r++) {
                const int src = L - 3 + r;
                hv[r] = src >= 0 ? big[(size_t)src * sh.stride + ch] : old[(size_t)(src + 3) * C + ch];
            }
#pragma unroll
            for (int r = 0; r < 3; r++) hist[(size_t)r * C + ch] = hv[r];
        }
    }
}

// Sequential over chunks for one head and 16 value columns, in two roles of 4 waves each.  The
// state role (waves 0-3) carries the recurrence: V' = U - W S, then S <- e^(G_last) S + KgT V';
// the output role (waves 4-7) computes o = Qg S + Qk V' from the same chunk's S and V'.  Both
// pass the same two LDS barriers per chunk: after the first, S of chunk c is in St[p]; between
// the two, the state role forms W S and V' while the output role forms Qg S; after the second, the
// state role forms KgT V' and writes chunk c + 1's S into St[p ^ 1] while the output role adds
// Qk V' and stores o.  So o's products and operand loads run beside the recurrence instead of on
// its chain, and each role's CU time goes to its own half of the chunk's operands.  Wave w of a
// role owns rows 16w..16w+15 of the chunk (and the state role state rows 32w..32w+31 for the
// update).  The arithmetic of every product is the single-role form's: the same split operands,
// the same three-chain MFMA sums in the same order.
constexpr int SCAN_T = 512;
__global__ __launch_bounds__(SCAN_T) void k_gdn_scan(const uint32_t* __restrict__ lu, const uint32_t* __restrict__ seqt,
                                                     const uint32_t* __restrict__ chunkt, float* __restrict__ state,
                                                     int L, int load_default, size_t state_off, float* __restrict__ o,
                                                     const f16* __restrict__ big, f16* hist, size_t hist_off, GdnShape sh,
                                                     GdnWs ws) {
    constexpr int DK = 128, DV = 128;
    constexpr int SP = DK + 4, VP = CH + 4;
    __shared__ __attribute__((aligned(16))) float St[2][DVS * SP];  // S^T: [column][k], chunk parity p
    __shared__ __attribute__((aligned(16))) float Vt[DVS * VP];     // V'^T: [column][token]
    const int tid = threadIdx.x, lane = tid & 63, w8 = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int role = w8 >> 2, wv = w8 & 3;
    const int fr = lane & 15, fg = lane >> 4;
    const int h = blockIdx.x, sl = blockIdx.y, H = sh.H, q = blockIdx.z;
    // The lu fields and the sequence's chunk range in one batch of scalar loads, issued before any
    // branch: the pointers are selected first, with `state` standing in for a null table (values
    // then unused).
    const uint32_t* lp = lu ? lu : reinterpret_cast<const uint32_t*>(state);
    const uint32_t* sp = seqt ? seqt + q : lp;
    const uint32_t lu_nseq = lp[5], lu_load = lp[3], se = *sp;
    const uint8_t* const lu_pre = *reinterpret_cast<const uint8_t* const*>(lp + 8);
    SGPR_BATCH("s"(lu_nseq), "s"(lu_load), "s"(se), "s"(lu_pre), "s"(hist), "s"(hist_off));
    if (seqt && q >= (int)lu_nseq) return;  // the grid is sized for the most sequences
    const int c0 = sl * DVS;
    const bool load = lu ? lu_load != 0u : load_default != 0;
    const uint8_t* pre = lu ? lu_pre : nullptr;
    float* Sg = state + (size_t)h * DK * DV;  // the live state (written back by a single sequence)
    const float* S0 = (pre ? reinterpret_cast<const float*>(pre + state_off) : state) + (size_t)h * DK * DV;
    {
        // The slice through a buffer resource, every load issued before the first LDS store (a load
        // under a branch, or a flat one, would be waited for before the next is issued); a fresh
        // state gets an empty resource, whose loads return 0 without touching memory.
        static_assert(DK * DVS % SCAN_T == 0, "whole passes of the workgroup");
        const Rsrc rs = make_rsrc(S0, load ? (uint32_t)(DK * DV * 4) : 0u);
        float sv[DK * DVS / SCAN_T];
#pragma unroll
        for (int i = 0; i < DK * DVS / SCAN_T; i++) {
            const int e = tid + SCAN_T * i, k = e / DVS, cc = e % DVS;
            sv[i] = __builtin_bit_cast(float, buf_b32(rs, (uint32_t)((k * DV + c0 + cc) * 4), 0u));
        }
#pragma unroll
        for (int i = 0; i < DK * DVS / SCAN_T; i++) {
            const int e = tid + SCAN_T * i, k = e / DVS, cc = e % DVS;
            St[0][cc * SP + k] = sv[i];
        }
    }
    // the reference's hist_update (src/kernels.rs:173-190): the last 3 rows of (the prefix's history
    // ++ this forward's rows) become the live history, each workgroup on a slice of the channels;
    // here, after the prep that read the old history for its conv.  This thread's channel lo + tid
    // is loaded now, before any store, and stored at the end (a longer slice loops there).
    const int hC = sh.C, hnb = H * (DV / DVS), hper = (hC + hnb - 1) / hnb;
    const int hlo = (blockIdx.y * H + h) * hper, hhi = min(hC, hlo + hper);
    const f16* hold = pre ? reinterpret_cast<const f16*>(pre + hist_off) : hist;
    f16 hv[3] = {};
    if (hist && hlo + tid < hhi) {
#pragma unroll
        for (int r = 0; r < 3; r++) {
            const int src = L - 3 + r;
            hv[r] = src >= 0 ? big[(size_t)src * sh.stride + hlo + tid] : hold[(size_t)(src + 3) * hC + hlo + tid];
        }
    }
    const int cfirst = seqt ? (int)(se & 0xFFFFu) : 0;
    const int cend = seqt ? cfirst + (int)(se >> 16) : (L + CH - 1) / CH;
    // A chunk's operands (prep's output, not written here) are loaded ahead of their use, each by
    // the role that uses it: W (state) and Qg (output) of chunk c + 1 into a second register set
    // during chunk c's first half, U of chunk c + 1 at chunk c's start; Kg and e^(G_last) (state)
    // and Qk (output) once chunk c has used its own.  Vector memory operations retire in issue
    // order (vmcnt), so the output role's o stores are issued after its loads: a wait for the loads
    // never waits for the stores to be acked.  e^(G_last) is a vector load too, so no scalar load is
    // outstanding at an LDS barrier.
    struct WS {  // state role
        f16x8 wh[4], wl[4];
        float ur[4];
    };
    struct QS {  // output role
        f16x8 qh[4], ql[4];
    };
    // The workspace is one allocation (W | Qg | Qk | Kg | U | e^G_last regions): every operand load
    // is a buffer load of it with this lane's fixed offset in a VGPR and the region, slot and
    // fragment offsets in SGPRs, so no per-load address arithmetic runs on the VALU.
    const uint8_t* wsb = reinterpret_cast<const uint8_t*>(ws.wf);
    const Rsrc rws = make_rsrc(wsb, 0x7FFFFFF0u);  // every offset below lies inside the workspace
    const uint32_t o_qg = (uint32_t)(reinterpret_cast<const uint8_t*>(ws.qgf) - wsb),
                   o_qk = (uint32_t)(reinterpret_cast<const uint8_t*>(ws.qkf) - wsb),
                   o_kg = (uint32_t)(reinterpret_cast<const uint8_t*>(ws.kgf) - wsb),
                   o_u = (uint32_t)(reinterpret_cast<const uint8_t*>(ws.u) - wsb),
                   o_gl = (uint32_t)(reinterpret_cast<const uint8_t*>(ws.gl) - wsb);
    const uint32_t vfrag = (uint32_t)lane * 16u;             // fragment layout
    const uint32_t vu = (uint32_t)((fg * 4 * DV + fr) * 4);  // U rows fg*4 + r, column fr
    // Every chunk issues the same loads with no branch around any of them: a chunk past the last
    // one gets out-of-range offsets (zeros, no memory access).  The compiler then counts exactly
    // which loads a wait must cover; a load under a branch leaves it unsure and it waits for more.
    auto slot_of = [&](int c) { return (uint32_t)((c < cend ? c : cfirst) * H + h); };
    auto frag = [&](uint32_t region, int KS, int rt, int s, f16x8& hi, f16x8& lo, uint32_t vf) {
        const uint32_t so = region + (uint32_t)((rt * KS + s) * 2) * 1024u;
        hi = __builtin_bit_cast(f16x8, buf_b128(rws, vf, so));
        lo = __builtin_bit_cast(f16x8, buf_b128(rws, vf, so + 1024u));
    };
    // S^T slice of k step s for this lane (column fr, k = 32 s + 8 fg ..), from St[p]
    auto s_slice = [&](int p, int s, float* v8) {
        const float* spp = &St[p][fr * SP + s * 32 + fg * 8];
#pragma unroll
        for (int u = 0; u < 8; u++) v8[u] = spp[u];
    };
    // V'^T fragments (B operand) of the chunk, both k steps
    auto v_frags = [&](f16x8 (&vh)[2], f16x8 (&vl)[2]) {
#pragma unroll
        for (int s = 0; s < 2; s++) {
            float v8[8];
            const float* vp = &Vt[fr * VP + s * 32 + fg * 8];
#pragma unroll
            for (int u = 0; u < 8; u++) v8[u] = vp[u];
            split8(v8, vh[s], vl[s]);
        }
    };
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    int c = cfirst;
    if (role == 0) {
        // ---- state role: V' = U - W S; S <- e^(G_last) S + KgT V'
        WS set0, set1;
        f16x8 kh[2][2], kl[2][2];
        float gl = 0.f;
        auto load_w_step = [&](WS& d, int cc, int s) {
            const uint32_t vf = cc < cend ? vfrag : OOB;
            frag(slot_of(cc) * (uint32_t)(WF_H * 2), 4, wv, s, d.wh[s], d.wl[s], vf);
        };
        auto load_u = [&](WS& d, int cc) {
            const uint32_t vuu = cc < cend ? vu : OOB, slot = slot_of(cc);
#pragma unroll
            for (int r = 0; r < 4; r++)
                d.ur[r] = __builtin_bit_cast(
                    float, buf_b32(rws, vuu, o_u + slot * (uint32_t)(U_F * 4) + (uint32_t)(((wv * 16 + r) * DV + c0) * 4)));
        };
        auto load_gl = [&](int cc) { gl = __builtin_bit_cast(float, buf_b32(rws, cc < cend ? 0u : OOB, o_gl + slot_of(cc) * 4u)); };
        auto load_kg = [&](int cc, int q2) {
            const uint32_t vf = cc < cend ? vfrag : OOB, slot = slot_of(cc);
#pragma unroll
            for (int s = 0; s < 2; s++)
                frag(o_kg + slot * (uint32_t)(KGF_H * 2), 2, wv * 2 + q2, s, kh[q2][s], kl[q2][s], vf);
        };
        auto chunk = [&](int cc, int p, const WS& cur, WS& nxt) {
            load_u(nxt, cc + 1);
            lds_barrier();  // St[p] holds this chunk's starting state; Vt is free
            f32x4 av[3] = {z4, z4, z4};
            // k step s: its S slice (read from LDS during step s - 1), then the next chunk's W loads
            // of step s, each step a scheduling region of its own so that those loads are issued
            // in four groups
            float sn[8];
            s_slice(p, 0, sn);
#pragma unroll
            for (int s = 0; s < 4; s++) {
                float s8[8];
#pragma unroll
                for (int u = 0; u < 8; u++) s8[u] = sn[u];
                if (s < 3) s_slice(p, s + 1, sn);
                load_w_step(nxt, cc + 1, s);
                f16x8 sh8, sl8;
                split8(s8, sh8, sl8);
                mma3s(cur.wh[s], cur.wl[s], sh8, sl8, av);
                __builtin_amdgcn_sched_barrier(0);
            }
            // rows wv * 16 + fg * 4 .. + 3 of column fr: one 16-byte store (conflict-free at this pitch)
            *reinterpret_cast<float4*>(&Vt[fr * VP + wv * 16 + fg * 4]) =
                float4{cur.ur[0] - (av[0][0] + av[1][0] + av[2][0]), cur.ur[1] - (av[0][1] + av[1][1] + av[2][1]),
                       cur.ur[2] - (av[0][2] + av[1][2] + av[2][2]), cur.ur[3] - (av[0][3] + av[1][3] + av[2][3])};
            lds_barrier();  // V' complete
            f16x8 vh[2], vl[2];
            v_frags(vh, vl);
            const float g_c = gl;
            load_gl(cc + 1);  // e^(G_last) is consumed
            // S <- e^(G_last) S + KgT V': state row tiles 2w, 2w+1
            f32x4 as[2][3];
#pragma unroll
            for (int q2 = 0; q2 < 2; q2++) {
                as[q2][0] = as[q2][1] = as[q2][2] = z4;
#pragma unroll
                for (int s = 0; s < 2; s++) mma3s(kh[q2][s], kl[q2][s], vh[s], vl[s], as[q2]);
                load_kg(cc + 1, q2);  // Kg row tile q2 is consumed
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int q2 = 0; q2 < 2; q2++) {
                // state rows k0 .. k0 + 3 of column fr: one 16-byte read of S_c and one write of S_c+1
                const int so = fr * SP + (wv * 2 + q2) * 16 + fg * 4;
                const float4 s4 = *reinterpret_cast<const float4*>(&St[p][so]);
                *reinterpret_cast<float4*>(&St[p ^ 1][so]) =
                    float4{g_c * s4.x + (as[q2][0][0] + as[q2][1][0] + as[q2][2][0]),
                           g_c * s4.y + (as[q2][0][1] + as[q2][1][1] + as[q2][2][1]),
                           g_c * s4.z + (as[q2][0][2] + as[q2][1][2] + as[q2][2][2]),
                           g_c * s4.w + (as[q2][0][3] + as[q2][1][3] + as[q2][2][3])};
            }
        };
#pragma unroll
        for (int s = 0; s < 4; s++) load_w_step(set0, cfirst, s);
        load_u(set0, cfirst);
        load_gl(cfirst);
        load_kg(cfirst, 0);
        load_kg(cfirst, 1);
        for (; c + 1 < cend; c += 2) {  // no branch inside the loop body
            chunk(c, 0, set0, set1);
            chunk(c + 1, 1, set1, set0);
        }
        if (c < cend) chunk(c, 0, set0, set1);
    } else {
        // ---- output role: o = Qg S + Qk V'
        QS set0, set1;
        f16x8 qkh[2], qkl[2];
        auto load_q_step = [&](QS& d, int cc, int s) {
            const uint32_t vf = cc < cend ? vfrag : OOB;
            frag(o_qg + slot_of(cc) * (uint32_t)(QGF_H * 2), 4, wv, s, d.qh[s], d.ql[s], vf);
        };
        auto load_qk = [&](int cc) {
            const uint32_t vf = cc < cend ? vfrag : OOB, slot = slot_of(cc);
#pragma unroll
            for (int s = 0; s < 2; s++) frag(o_qk + slot * (uint32_t)(QKF_H * 2), 2, wv, s, qkh[s], qkl[s], vf);
        };
        // o rows t0 + wv*16 + fg*4 + r (r < 4), column h*DV + c0 + fr; rows past the chunk get an
        // out-of-range offset and are not written
        const Rsrc ro = make_rsrc(o, (uint32_t)L * sh.H * DV * 4);
        const uint32_t vo = (uint32_t)((fg * 4 * sh.H * DV + fr) * 4);
        auto chunk = [&](int cc, int p, const QS& cur, QS& nxt) {
            const int t0 = chunkt ? (int)(chunkt[cc] & 0xFFFFu) : cc * CH;
            const int Lc = chunkt ? (int)(chunkt[cc] >> 16) : min(CH, L - cc * CH);
            lds_barrier();  // St[p] holds this chunk's starting state
            f32x4 ao[3] = {z4, z4, z4};
            float sn[8];
            s_slice(p, 0, sn);
#pragma unroll
            for (int s = 0; s < 4; s++) {
                float s8[8];
#pragma unroll
                for (int u = 0; u < 8; u++) s8[u] = sn[u];
                if (s < 3) s_slice(p, s + 1, sn);
                load_q_step(nxt, cc + 1, s);
                f16x8 sh8, sl8;
                split8(s8, sh8, sl8);
                mma3s(cur.qh[s], cur.ql[s], sh8, sl8, ao);
                __builtin_amdgcn_sched_barrier(0);
            }
            lds_barrier();  // V' complete
            f16x8 vh[2], vl[2];
            v_frags(vh, vl);
#pragma unroll
            for (int s = 0; s < 2; s++) mma3s(qkh[s], qkl[s], vh[s], vl[s], ao);
            load_qk(cc + 1);  // Qk is consumed
            __builtin_amdgcn_sched_barrier(0);
            const uint32_t so = (uint32_t)(((t0 + wv * 16) * sh.H * DV + h * DV + c0) * 4);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const bool in = wv * 16 + fg * 4 + r < Lc;
                buf_st32(ro, in ? vo + (uint32_t)(r * sh.H * DV * 4) : OOB, so,
                         __builtin_bit_cast(uint32_t, ao[0][r] + ao[1][r] + ao[2][r]));
            }
        };
#pragma unroll
        for (int s = 0; s < 4; s++) load_q_step(set0, cfirst, s);
        load_qk(cfirst);
        for (; c + 1 < cend; c += 2) {
            chunk(c, 0, set0, set1);
            chunk(c + 1, 1, set1, set0);
        }
        if (c < cend) chunk(c, 0, set0, set1);
    }
    if (seqt) return;  // several sequences: their final states are not kept
    __syncthreads();
    const int pf = (cend - cfirst) & 1;  // the buffer holding the final state
    for (int e = tid; e < DK * DVS; e += SCAN_T) {
        const int k = e / DVS, cc = e % DVS;
        Sg[k * DV + c0 + cc] = St[pf][cc * SP + k];
    }
    if (hist) {
        if (hlo + tid < hhi) {
#pragma unroll
            for (int r = 0; r < 3; r++) hist[(size_t)r * hC + hlo + tid] = hv[r];
        }
        for (int ch = hlo + tid + SCAN_T; ch < hhi; ch += SCAN_T) {
            f16 v3[3];
#pragma unroll
            for (int r = 0; r < 3; r++) {
                const int src = L - 3 + r;
                v3[r] = src >= 0 ? big[(size_t)src * sh.stride + ch] : hold[(size_t)(src + 3) * hC + ch];
            }
#pragma unroll
            for (int r = 0; r < 3; r++) hist[(size_t)r * hC + ch] = v3[r];
        }
    }
}

// out[t, h*DV + c] = f16(w[c] o rsqrt(mean(o^2) + 1e-6) silu(z)); one wave per (t, h), DV = 128.
__global__ __launch_bounds__(256) void k_gnorm(const float* __restrict__ o, const f16* __restrict__ big,
                                               const float* __restrict__ w, f16* __restrict__ out, int L, int H,
                                               int DV, int stride, int z_off) {
    const struct { int H, DV, stride, z_off; } sh{H, DV, stride, z_off};
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= L * sh.H) return;
    const int t = row / sh.H, h = row % sh.H;
    // lane: the two consecutive values 2 lane, 2 lane + 1 (8- and 4-byte accesses)
    const size_t b = (size_t)t * sh.H * sh.DV + h * sh.DV + 2 * lane;
    const float2 v = *reinterpret_cast<const float2*>(o + b);
    float ss = v.x * v.x + v.y * v.y;
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) ss += __shfl_xor(ss, s);
    const float inv = 1.0f / sqrtf(ss / (float)sh.DV + 1e-6f);
    const f16x2 z = *reinterpret_cast<const f16x2*>(big + (size_t)t * sh.stride + sh.z_off + h * sh.DV + 2 * lane);
    const float2 w2 = *reinterpret_cast<const float2*>(w + 2 * lane);
    const float z0 = (float)z[0], z1 = (float)z[1];
    const f16x2 r = {(f16)(w2.x * v.x * inv * z0 / (1.0f + expf(-z0))), (f16)(w2.y * v.y * inv * z1 / (1.0f + expf(-z1)))};
    *reinterpret_cast<f16x2*>(out + b) = r;
}

// The same with 16 lanes per (t, h) row, 8 values each: 16-byte loads of o, z and w and one 16-byte
// store, 16 rows per workgroup (z_off and stride multiples of 8).  The sum of squares runs over the
// lane's 8 values, then over the 16 lanes of the row.
__global__ __launch_bounds__(256) void k_gnorm8(const float* __restrict__ o, const f16* __restrict__ big,
                                                const float* __restrict__ w, f16* __restrict__ out, int L, int H,
                                                int stride, int z_off) {
    constexpr int DV = 128;
    const int row = blockIdx.x * 16 + (threadIdx.x >> 4);
    const int l16 = threadIdx.x & 15;
    if (row >= L * H) return;  // a row's 16 lanes exit together; the shuffles stay inside the row
    const int t = row / H, h = row % H;
    const size_t b = (size_t)t * H * DV + h * DV + 8 * l16;
    const float4 v0 = *reinterpret_cast<const float4*>(o + b), v1 = *reinterpret_cast<const float4*>(o + b + 4);
    const f16x8 z = *reinterpret_cast<const f16x8*>(big + (size_t)t * stride + z_off + h * DV + 8 * l16);
    const float4 w0 = *reinterpret_cast<const float4*>(w + 8 * l16), w1 = *reinterpret_cast<const float4*>(w + 8 * l16 + 4);
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < 8; u++) ss += v[u] * v[u];
#pragma unroll
    for (int s = 8; s > 0; s >>= 1) ss += __shfl_xor(ss, s);
    const float inv = 1.0f / sqrtf(ss / (float)DV + 1e-6f);
    f16x8 r;
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const float zu = (float)z[u];
        r[u] = (f16)(wv[u] * v[u] * inv * zu / (1.0f + expf(-zu)));
    }
    *reinterpret_cast<f16x8*>(out + b) = r;
}

}  // namespace

// Room for the chunks of `cap` rows split into up to SD_MAX_SEQS sequences.
size_t gdn_ws_bytes(int cap, const GdnShape& s) {
    const size_t slots = (size_t)((cap + CH - 1) / CH + SD_MAX_SEQS) * s.H;
    return slots * ((WF_H + QGF_H + QKF_H + KGF_H) * 2 + (U_F + 1) * 4) + 1024;
}

void gdn_ws_carve(void* base, int cap, const GdnShape& s, GdnWs& ws) {
    const size_t slots = (size_t)((cap + CH - 1) / CH + SD_MAX_SEQS) * s.H;
    f16* p = static_cast<f16*>(base);
    ws.wf = p;
    ws.qgf = ws.wf + slots * WF_H;
    ws.qkf = ws.qgf + slots * QGF_H;
    ws.kgf = ws.qkf + slots * QKF_H;
    ws.u = reinterpret_cast<float*>(ws.kgf + slots * KGF_H);
    ws.gl = ws.u + slots * U_F;
}

void conv_silu(const f16* big, int stride, int L, int C, const float* w, const f16* hist, float* out, const Segs& sg,
               hipStream_t st, const uint32_t* lu, size_t hist_off) {
    SD_CHECK(C % 4 == 0 && stride % 4 == 0, "conv: channels and row stride must be multiples of 4");
    // rows per workgroup: enough workgroups to fill the chip, at most 8 rows each
    const int cb = (C / 4 + 255) / 256;
    int R = 1;
    while (R < 8 && (size_t)cb * ((L + 2 * R - 1) / (2 * R)) >= 512) R *= 2;
    hipLaunchKernelGGL(k_conv, dim3(cb, (L + R - 1) / R), dim3(256), 0, st, big, stride, L, C, w, hist, out, sg.row, R, lu,
                       hist_off);
    launched("conv");
}

void gdn_prep(const float* qkvc, const f16* big, const GdnShape& s, const float* negA, const float* dtb, int L,
              const GdnWs& ws, const ConvIn& cv, const Segs& sg, int nch, const uint32_t* lu, hipStream_t st) {
    SD_CHECK(s.DK == 128 && s.DV == 128, "gated delta net: only 128-wide key/value heads are supported");
    SD_CHECK(!sg.chunk || lu, "gdn_prep: several sequences need lu");
    SD_CHECK(!cv.w || cv.hist, "gdn_prep: the conv needs the history");
    SD_CHECK(!cv.w || (s.C % 4 == 0 && s.stride % 4 == 0), "gdn_prep: channels and row stride must be multiples of 4");
    if (!sg.chunk) nch = (L + CH - 1) / CH;
    const dim3 grid(nch, s.H, 2);
    if (cv.w)
        hipLaunchKernelGGL(k_gdn_prep<true>, grid, dim3(PREP_T), 0, st, sg.chunk, lu, big, qkvc, negA, dtb, L, s, ws, cv);
    else
        hipLaunchKernelGGL(k_gdn_prep<false>, grid, dim3(PREP_T), 0, st, sg.chunk, lu, big, qkvc, negA, dtb, L, s, ws, cv);
    launched("gdn_prep");
}

void gdn_scan(const GdnShape& s, int L, const GdnWs& ws, float* state, const uint32_t* lu, int load_default, float* o,
              const Segs& sg, int nseq, hipStream_t st, size_t state_off, f16* hist, const f16* big, size_t hist_off) {
    SD_CHECK(s.DK == 128 && s.DV == 128, "gated delta net: only 128-wide key/value heads are supported");
    SD_CHECK(!sg.seq || (lu && sg.chunk), "gdn_scan: several sequences need lu and the chunk table");
    SD_CHECK(!hist || (!sg.seq && big), "gdn_scan: the history update needs one sequence and big");
    if (!sg.seq) nseq = 1;
    hipLaunchKernelGGL(k_gdn_scan, dim3(s.H, s.DV / DVS, nseq), dim3(SCAN_T), 0, st, lu, sg.seq, sg.chunk, state, L,
                       load_default, state_off, o, big, hist, hist_off, s, ws);
    launched("gdn_scan");
}

void gdn_recur(const float* qkvc, const f16* big, const GdnShape& s, const float* negA, const float* dtb, int L,
               float* state, const uint32_t* lu, int load_default, float* o, f16* hist, const Segs& sg, int nseq,
               hipStream_t st, size_t state_off, size_t hist_off, const ConvIn& cv) {
    SD_CHECK(s.DK == 128 && s.DV == 128, "gated delta net: only 128-wide key/value heads are supported");
    SD_CHECK(!sg.seq || (lu && sg.chunk && !hist), "gdn_recur: several sequences need lu and keep no history");
    SD_CHECK(!cv.w || (cv.hist && !hist), "gdn_recur: the conv needs the history, and updates none");
    SD_CHECK(!cv.w || (s.C % 4 == 0 && s.stride % 4 == 0), "gdn_recur: channels and row stride must be multiples of 4");
    if (!sg.seq) nseq = 1;
    if (cv.w)
        hipLaunchKernelGGL(k_gdn_recur<true>, dim3(s.H, s.DV / RC, nseq), dim3(RT), 0, st, lu, sg.seq, state, big, qkvc,
                           L, load_default, state_off, negA, dtb, o, sg.chunk, hist, hist_off, s, cv);
    else
        hipLaunchKernelGGL(k_gdn_recur<false>, dim3(s.H, s.DV / RC, nseq), dim3(RT), 0, st, lu, sg.seq, state, big, qkvc,
                           L, load_default, state_off, negA, dtb, o, sg.chunk, hist, hist_off, s, cv);
    launched("gdn_recur");
}

void gnorm(const float* o, const f16* big, const GdnShape& s, const float* w, int L, f16* out, hipStream_t st) {
    SD_CHECK(s.DV == 128, "gnorm: only 128-wide value heads are supported");
    SD_CHECK(s.stride % 2 == 0 && s.z_off % 2 == 0, "gnorm: gate row stride and offset must be even");
    const int rows = L * s.H;
    if (s.stride % 8 == 0 && s.z_off % 8 == 0)
        hipLaunchKernelGGL(k_gnorm8, dim3((rows + 15) / 16), dim3(256), 0, st, o, big, w, out, L, s.H, s.stride, s.z_off);
    else
        hipLaunchKernelGGL(k_gnorm, dim3((rows + 3) / 4), dim3(256), 0, st, o, big, w, out, L, s.H, s.DV, s.stride, s.z_off);
    launched("gnorm");
}

}  // namespace sd
