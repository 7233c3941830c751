// Full-attention sublayer on gfx950: q/k RMSNorm + partial rotate-half RoPE with the K/V cache
// write (reference: src/kernels.rs:400-448), and causal GQA attention with a sigmoid output gate
// (reference: src/kernels.rs:453-541).
//
// Attention runs on MFMA (k_attn below).  When the query blocks alone cannot fill the GPU (the
// short question suffix over a long cached prefix), the key range is also split over workgroups
// and a combine kernel merges the partial (max, sum, acc).  As in the reference, q is pre-scaled
// by 1/sqrt(hd) and rounded to f16 before the dot products.  The cache is kept in blocks of 32
// keys, so that the fragment loads of a key block touch whole cache lines: K as [hk][ctx / 32]
// [hd / 32][32 keys][32 dims] (a load of 16 keys x 8 dims reads pairs of consecutive keys' 64 bytes),
// V transposed as [hk][ctx / 32][hd][32 keys] (a block's V^T is 16 KB of consecutive bytes).
#include <climits>
#include <cmath>

#include "common.h"
#include "device.h"

namespace sd {
namespace {

constexpr int BQ = 16;  // queries per workgroup
constexpr int ATTN_KS_MAX = 8;  // key splits the workspace and k_attn_combine provide for

// Kernel arguments: what the prologue needs first, and the head shape as ints, lead (the first 16
// dwords are preloaded into SGPRs, up to the first struct argument).
template <int HD>
__global__ __launch_bounds__(256) void k_qk_prep(const f16* __restrict__ big, const uint32_t* __restrict__ lu, int L,
                                                 int HQ, int HK, int RD, int stride, int ctx,
                                                 const uint32_t* __restrict__ rowt, const float* __restrict__ qw,
                                                 const float* __restrict__ kw, const float* __restrict__ rope,
                                                 f16* __restrict__ Q, f16* __restrict__ Kc, f16* __restrict__ Vc) {
    const AttnShape s{HQ, HK, HD, RD, stride, ctx};
    // Workgroup (4 rows, one q or kv head): wave w takes row w, lane l the 4 dimensions 4l..4l+3
    // (8-byte loads and stores, the norm a wave reduction).  A kv head also writes the 4 rows of
    // V^T, dimension by dimension: 8 contiguous bytes per dimension.
    static_assert(HD == 256, "qk_prep is written for 256-wide heads");
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // without Q the grid covers the kv heads only (the attention kernel computes its queries itself)
    const int t0 = blockIdx.x * 4, slot = Q ? (int)blockIdx.y : s.HQ + (int)blockIdx.y;
    const int P = (int)lu[1];
    const bool isq = slot < s.HQ;
    const int k_off = 2 * s.HQ * HD, v_off = k_off + s.HK * HD;
    const int nt = min(4, L - t0);
    if (!isq) {  // V^T in 32-key blocks, [hk][ctx / 32][hd][32]: thread d writes rows t0 .. t0+3
        const int kh = slot - s.HQ, d = tid;
        f16 v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = i < nt ? big[(size_t)(t0 + i) * s.stride + v_off + kh * HD + d] : (f16)0.f;
        auto at = [&](int pos) { return Vc + (((size_t)kh * (s.ctx / 32) + pos / 32) * HD + d) * 32 + pos % 32; };
        if (nt == 4 && ((P + t0) & 3) == 0) {  // the 4 rows lie in one block
            *reinterpret_cast<f16x4*>(at(P + t0)) = f16x4{v[0], v[1], v[2], v[3]};
        } else {
            for (int i = 0; i < nt; i++) *at(P + t0 + i) = v[i];
        }
    }
    __shared__ __align__(16) float nrow[4][HD];  // a wave's normalized row (rotary dims not a multiple of 8)
    const float* nw = isq ? qw : kw;
    const float4 w4 = *reinterpret_cast<const float4*>(nw + 4 * lane);
    const int rd2 = s.RD / 2;
    if (wv < nt) {
        const int t = t0 + wv;
        const int pos = P + t;                                        // cache row
        const int rpos = P + (rowt ? (int)(rowt[t] & 0xFFFFu) : t);  // RoPE position
        const f16* src = big + (size_t)t * s.stride + (isq ? slot * 2 * HD : k_off + (slot - s.HQ) * HD) + 4 * lane;
        const f16x4 x4 = *reinterpret_cast<const f16x4*>(src);
        float x[4] = {(float)x4[0], (float)x4[1], (float)x4[2], (float)x4[3]};
        float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
        const float inv = 1.0f / sqrtf(ss / (float)HD + 1e-6f);
        const float wv4[4] = {w4.x, w4.y, w4.z, w4.w};
        float n[4];
#pragma unroll
        for (int u = 0; u < 4; u++) n[u] = x[u] * inv * wv4[u];
        // rotate-half RoPE on dims < RD: the partner of dim d is d +- RD/2.  With RD a multiple of 8
        // it is element u of lane l +- RD/8 (a lane shuffle); otherwise it is read back from the
        // wave's row in LDS (the wave's own stores: LDS operations of one wave complete in order).
        float pn[4];
        if (rd2 % 4 == 0) {
            const int sh = rd2 / 4;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float up = __shfl(n[u], (lane + sh) & 63), dn = __shfl(n[u], (lane - sh) & 63);
                pn[u] = 4 * lane < rd2 ? up : dn;
            }
        } else {
            *reinterpret_cast<float4*>(&nrow[wv][4 * lane]) = float4{n[0], n[1], n[2], n[3]};
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int d = 4 * lane + u;
                pn[u] = d < s.RD ? nrow[wv][d < rd2 ? d + rd2 : d - rd2] : 0.f;
            }
        }
        f16x4 r4;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int d = 4 * lane + u;
            float r = n[u];
            if (d < s.RD) {
                const int j = d % rd2;
                const float c = rope[((size_t)rpos * rd2 + j) * 2], sn = rope[((size_t)rpos * rd2 + j) * 2 + 1];
                r = d < rd2 ? n[u] * c - pn[u] * sn : n[u] * c + pn[u] * sn;
            }
            r4[u] = (f16)r;
        }
        if (isq) *reinterpret_cast<f16x4*>(Q + ((size_t)slot * L + t) * HD + 4 * lane) = r4;
        else
            *reinterpret_cast<f16x4*>(Kc + (((size_t)(slot - s.HQ) * (s.ctx / 32) + pos / 32) * (HD / 32) + lane / 8) * 1024 +
                                      (pos % 32) * 32 + 4 * (lane % 8)) = r4;
    }
}

// The online softmax runs in base 2: scores are scaled by log2(e) and exponentiated with
// v_exp_f32, exp(s - m) = 2^(s log2 e - m log2 e); max and sum states (also those the combine kernel
// merges) are in these units.
constexpr float LOG2E = 1.4426950408889634f;
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float wave_max16(float v) {  // max over lanes {l, l^16, l^32, l^48}
    v = fmaxf(v, __shfl_xor(v, 16));
    return fmaxf(v, __shfl_xor(v, 32));
}
__device__ __forceinline__ float wave_sum16(float v) {
    v += __shfl_xor(v, 16);
    return v + __shfl_xor(v, 32);
}

// Causal GQA attention on MFMA.  A workgroup takes 16 queries of one q head; its 4 waves split the
// key range in blocks of 32 keys (wave w takes blocks w, w+4, ...) and merge their online-softmax
// states in LDS at the end.  Per 32-key block a wave computes S^T = K Q^T (keys x queries, 2 x 8
// v_mfma_f32_16x16x32_f16 over the 256 dims), the online softmax per query (column), then
// O^T += V^T P^T (256 dims x 16 queries); with S^T in the MFMA output layout, P^T is already in
// the B-operand layout (lane = query, 8 keys), and the V cache is stored transposed so V^T
// fragments are contiguous (the keys of a block are permuted so that they are 8 consecutive).  P is
// split into f16 hi + lo (two MFMAs) so that the product keeps the reference's f32 P.V to about 22
// bits.  With ks > 1 the workgroups along z also split the keys
// and write unnormalised (acc, max, sum) for k_attn_combine.
template <int HD, int QRD>
__global__ __launch_bounds__(256) void k_attn(const f16* __restrict__ Q, const f16* __restrict__ Kc,
                                              const f16* __restrict__ Vt, const uint32_t* __restrict__ lu, int L,
                                              int HQ, int HK, int stride, int ctx, int ks,
                                              const uint32_t* __restrict__ rowt, const f16* __restrict__ big,
                                              f16* __restrict__ out, float* __restrict__ pacc, float* __restrict__ pml,
                                              const float* __restrict__ qw, const float* __restrict__ rope, int RD) {
    const AttnShape s{HQ, HK, HD, 0, stride, ctx};
    static_assert(HD == 256, "attention is written for 256-wide heads");
    constexpr int ND = HD / 16;   // 16 output dimension tiles
    constexpr int NS = HD / 32;   // 8 k steps over the head dimension
    constexpr int KB = 32;        // keys per block
    __shared__ float Om[4][16][HD + 4];  // per-wave unnormalised outputs [query][dim]
    __shared__ float Mm[4][16], Lm[4][16];
    __shared__ __align__(16) f16 Qs[16][HD + 8];  // the workgroup's queries, scaled (row padding: no bank conflicts on the fragment reads)
    // wv is wave-uniform (readfirstlane): the key loop below is then a scalar loop, not a divergent one
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int fq = lane & 15, fg = lane >> 4;
    // cache rows below Pv are every sequence's shared prefix: the cached prefix (P) and, in a forward
    // whose sequences continue one state sequence (lu[6] > 0), that state's rows too
    const int P = (int)lu[1], Pv = P + (int)lu[6];
    SGPR_BATCH("s"(P), "s"(Pv), "s"(rowt), "s"(big), "s"(out), "s"(pacc), "s"(pml));
    const int t0 = blockIdx.x * 16, h = blockIdx.y, z = blockIdx.z;
    const int kh = h / (s.HQ / s.HK);
    const int nq = min(16, L - t0);
    const int nkeys = P + t0 + nq;  // keys 0 .. P + t0 + nq - 1 can be attended
    const int span = ((nkeys + ks - 1) / ks + KB - 1) / KB * KB;
    const int kbeg = z * span, kend = min(nkeys, kbeg + span);
    const float scale = 1.0f / sqrtf((float)HD);
    const int qpos = P + t0 + fq;  // cache row of this lane's query
    const bool qok = fq < nq;
    // keys below jend can be attended by this lane's query (none past nq): the causal limit and the
    // split's end
    const int jend = qok ? min(kend, qpos + 1) : INT_MIN;
    // The row table words of this lane's query and of the tile's first row: buffer loads, issued
    // together and without a branch (a null table is a 0-byte buffer, whose loads read 0).
    const Rsrc rr = make_rsrc(rowt, rowt ? (uint32_t)L * 4u : 0u);
    const uint32_t rwq = buf_b32(rr, (uint32_t)(t0 + min(fq, nq - 1)) * 4u, 0);
    const uint32_t rw0 = buf_b32(rr, (uint32_t)t0 * 4u, 0);
    // and, for the fused query norm and RoPE, that of query 4 wv + lane / 16 (read for its position)
    const uint32_t rwp = QRD ? buf_b32(rr, (uint32_t)(t0 + min(4 * wv + (lane >> 4), nq - 1)) * 4u, 0) : 0u;
    // first cache row of the query's own sequence: rows [Pv, qlo) belong to other sequences
    const int qlo = P + (int)(rwq >> 16);
    // the tile's first row starts the earliest sequence among its queries: a key block inside
    // [Pv, qlo0) belongs to other sequences for every query, is wholly masked and is skipped (its
    // softmax update would leave the running max, sum and output unchanged)
    const int qlo0 = P + (int)(rw0 >> 16);

    // Q^T fragments (B operand), filled after the first key block's loads are issued
    f16x8 qf[NS];
    // The epilogue gives thread tid query qe = tid / 16 and the 16 dimensions d0 .. d0 + 15: its
    // output gates are loaded here (two 16-byte loads, unconditionally: queries past nq read the
    // last one's), while the keys are processed.
    const int qe = tid >> 4, d0 = (tid & 15) * 16;
    f16x8 gv[2];
    {
        const f16* gp = big + (size_t)(t0 + min(qe, nq - 1)) * s.stride + h * 2 * HD + HD + d0;
        gv[0] = *reinterpret_cast<const f16x8*>(gp);
        gv[1] = *reinterpret_cast<const f16x8*>(gp + 8);
    }
    f32x4 acc[ND];
#pragma unroll
    for (int dt = 0; dt < ND; dt++) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;
    const f16* Kb = Kc + (size_t)kh * s.ctx * HD;
    const f16* Vb = Vt + (size_t)kh * HD * s.ctx;

    // The wave's key blocks are kbeg + 32 wv + 128 n below kend; those wholly inside [Pv, qlo0) are
    // skipped.  A block's K and V fragments are loaded one block ahead, into the other of two
    // register sets, while the current block's MFMAs and softmax run (one wave per SIMD: no other
    // wave hides a block's load latency).  Every step issues the same 32 loads (past the end they
    // re-read the last block, never used), so the explicit vmcnt wait is exact.
    auto next_block = [&](int j) {
        if (j >= Pv && j + KB <= qlo0) j += ((qlo0 - KB - j) / (4 * KB) + 1) * (4 * KB);
        return j;
    };
    // Keys are ordered inside the 32-key block so that lane (query fq, group fg) ends up with the
    // probabilities of keys j0 + 8fg .. +7: row i of S^T tile tt is key j0 + 8(i/4) + 4tt + i%4.
    // Then the V^T fragment of lane (dim fq, group fg) is those 8 keys, one 16-byte load.
    // The loads of a block stay where they are issued, ahead of the block in flight: the compiler
    // would otherwise sink them to their first use, a block later.  A memory clobber alone does not
    // hold them (the cache pointers are restrict: no asm without them could write their memory), so
    // the clobbering asm takes both pointers as operands.
    const Rsrc rk = make_rsrc(Kb, (uint32_t)s.ctx * HD * 2u), rv = make_rsrc(Vb, (uint32_t)s.ctx * HD * 2u);
    // A block's K fragments (2 NS loads) and V fragments (ND loads).  Past the end they re-read the
    // last block (never used), so every block issues the same loads and the explicit vmcnt waits
    // below are exact.
    auto koff = [&](int j, int tt) {
        const int key = min(min(j, kend - 1) + 8 * (fq >> 2) + 4 * tt + (fq & 3), kend - 1);
        return (uint32_t)((key >> 5) * (HD * 32) + (key & 31) * 32 + fg * 8) * 2u;
    };
    auto voff = [&](int j) { return (uint32_t)((min(j, kend - 1) >> 5) * (HD * 32) + fq * 32 + fg * 8) * 2u; };
    // (the clobbering asm takes both pointers, so the loads before it stay before it)
    auto pin = [&]() {
        asm volatile("" ::"s"(Kb), "s"(Vb) : "memory");
        __builtin_amdgcn_sched_barrier(0);
    };
    // Block j0 with the fragments kf, vf, and block jn's loads into kfn, vfn, issued among block
    // j0's MFMAs (K among S = K Q^T, V among O += V^T P^T): the CU's vector memory path takes 64
    // bytes a clock, so a burst of a block's 32 KB per wave held up the wave's issue instead of
    // running beside its MFMAs.  A block's K is waited for before its S, its V before its P V.
    auto process = [&](int j0, const f16x8 (&kf)[2][NS], const f16x8 (&vf)[ND], int jn, f16x8 (&kfn)[2][NS],
                       f16x8 (&vfn)[ND]) {
        wait_loads<vmcnt_imm(ND)>();  // block j0's K has arrived (its V may still be in flight)
        f32x4 st2[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
        const uint32_t kn0 = koff(jn, 0), kn1 = koff(jn, 1);
#pragma unroll
        for (int st = 0; st < NS; st++) {
#pragma unroll
            for (int tt = 0; tt < 2; tt++) {
                st2[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[tt][st], qf[st], st2[tt], 0, 0, 0);
                kfn[tt][st] = __builtin_bit_cast(f16x8, buf_b128(rk, tt ? kn1 : kn0, (uint32_t)st * 2048u));
            }
        }
#pragma unroll
        for (int i = 0; i < 2 * NS; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one load
        }
        pin();
        float sv[8];
        float tmax = -INFINITY;
        // a block before every query of the workgroup (and, with several sequences, inside the
        // shared prefix) needs no mask; the rows of queries past nq are computed but never stored
        const bool open = j0 + KB <= kend && j0 + KB <= P + t0 + 1 && (!rowt || j0 + KB <= Pv);
#pragma unroll
        for (int tt = 0; tt < 2; tt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                // kept: below the lane's end and outside other sequences' rows (bitwise, not
                // short-circuit operators: the short-circuit form compiled to a branch per key)
                const int j = j0 + 8 * fg + 4 * tt + r;
                const bool keep = open | ((j < jend) & ((j < Pv) | (j >= qlo)));
                const float v = keep ? st2[tt][r] * LOG2E : -INFINITY;
                sv[tt * 4 + r] = v;
                tmax = fmaxf(tmax, v);
            }
        tmax = wave_max16(tmax);
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = m_run == -INFINITY ? 0.f : exp2_fast(m_run - m_new);
        const float m_sub = m_new == -INFINITY ? 0.f : m_new;  // every key masked so far: p = 2^-inf = 0
        float psum = 0.f;
        f16x8 ph, pl;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float pv = exp2_fast(sv[e] - m_sub);
            psum += pv;
            const f16 hi = (f16)pv;
            ph[e] = hi;
            pl[e] = (f16)(pv - (float)hi);
        }
        l_run = l_run * alpha + wave_sum16(psum);
        m_run = m_new;
        // O^T += V^T P^T
        wait_loads<vmcnt_imm(2 * NS)>();  // block j0's V has arrived (block jn's K may still be in flight)
        const uint32_t vn = voff(jn);
#pragma unroll
        for (int dt = 0; dt < ND; dt++) {
            f32x4 a = acc[dt];
            a[0] *= alpha, a[1] *= alpha, a[2] *= alpha, a[3] *= alpha;
            a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[dt], ph, a, 0, 0, 0);
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[dt], pl, a, 0, 0, 0);
            vfn[dt] = __builtin_bit_cast(f16x8, buf_b128(rv, vn, (uint32_t)dt * 1024u));
        }
#pragma unroll
        for (int i = 0; i < ND; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // two MFMAs
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one load
        }
        pin();
    };
    f16x8 kA[2][NS], vA[ND], kB[2][NS], vB[ND];
    // Q^T fragments: lane (query fq, group fg) holds Q[fq][32s + 8fg .. +8], pre-scaled by 1/sqrt(hd)
    // and rounded to f16 as the reference does.  The 4 waves prepare them together: wave w takes
    // queries 4w .. 4w + 3, lane (query qq, part kq) two 8-dim chunks c0, c1 of query qq, and writes
    // them to LDS, from where every wave reads its fragments.  Their loads are issued before the
    // first key block's and waited for alone (they are the older ones), so that the computation
    // runs while the block is in flight.
    //
    // QRD = RD: the query's RMSNorm and rotate-half RoPE are done here (the reference's qk_prep for
    // q, src/kernels.rs:400-448): q = x rsqrt(mean(x^2) + 1e-6) w, dims d < RD rotated at the row's
    // RoPE position, rounded to f16, then scaled.  Chunk c (dims 8c .. 8c + 7) of a rotated half
    // pairs with chunk c + NR: part kq < NR takes chunks kq and kq + NR (one cos/sin row for both),
    // part kq >= NR the unrotated chunks 2kq and 2kq + 1 (with QRD = 0 every part: dims 16kq ..
    // 16kq + 15 of the Q row).  The sum of squares is the 16 parts' (lanes 16 apart never mix).
    constexpr int RD2 = QRD / 2, NR = RD2 / 8;
    static_assert(QRD % 16 == 0 && QRD <= HD, "the fused query needs rotary_dim a multiple of 16");
    const int qq = 4 * wv + (lane >> 4), kq = lane & 15;
    const int tq = t0 + min(qq, nq - 1);
    const bool rot = kq < NR;
    const int c0 = rot ? kq : 2 * kq, c1 = rot ? kq + NR : 2 * kq + 1;
    f16x8 xv[2];
    float4 wq[2][2], cs4[4];
    if constexpr (QRD == 0) {
        const f16* qrow = Q + ((size_t)h * L + tq) * HD;
        xv[0] = *reinterpret_cast<const f16x8*>(qrow + 8 * c0);
        xv[1] = *reinterpret_cast<const f16x8*>(qrow + 8 * c1);
        // (the clobber holds the loads here: it takes the pointer, so it may write their memory)
        asm volatile("" ::"s"(Q) : "memory");
    } else {
        const f16* xrow = big + (size_t)tq * s.stride + h * 2 * HD;
        // unrotated parts read a rotated part's cos/sin row and do not use it
        xv[0] = *reinterpret_cast<const f16x8*>(xrow + 8 * c0);
        xv[1] = *reinterpret_cast<const f16x8*>(xrow + 8 * c1);
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int u = 0; u < 2; u++) wq[c][u] = *reinterpret_cast<const float4*>(qw + 8 * (c ? c1 : c0) + 4 * u);
        const int rpos = P + (rowt ? (int)(rwp & 0xFFFFu) : tq);
        const float* rp = rope + ((size_t)rpos * RD2 + 8 * (kq % NR)) * 2;
#pragma unroll
        for (int u = 0; u < 4; u++) cs4[u] = *reinterpret_cast<const float4*>(rp + 4 * u);
        asm volatile("" ::"s"(big), "s"(qw), "s"(rope) : "memory");
    }
    __builtin_amdgcn_sched_barrier(0);
    int j = next_block(kbeg + wv * KB);
    {
        // the first block's K, then V (the order process() waits in)
        const uint32_t k0 = koff(j, 0), k1 = koff(j, 1), v0 = voff(j);
#pragma unroll
        for (int tt = 0; tt < 2; tt++)
#pragma unroll
            for (int st = 0; st < NS; st++)
                kA[tt][st] = __builtin_bit_cast(f16x8, buf_b128(rk, tt ? k1 : k0, (uint32_t)st * 2048u));
#pragma unroll
        for (int dt = 0; dt < ND; dt++) vA[dt] = __builtin_bit_cast(f16x8, buf_b128(rv, v0, (uint32_t)dt * 1024u));
        pin();
    }
    {
        f16x8 q8[2];
        if constexpr (QRD == 0) {
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int e = 0; e < 8; e++) q8[c][e] = (f16)((float)xv[c][e] * scale);
        } else {
            float x[2][8], sp[2] = {0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    x[c][e] = (float)xv[c][e];
                    sp[c] += x[c][e] * x[c][e];
                }
            float ss = sp[0] + sp[1];
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) ss += __shfl_xor(ss, o);
            const float inv = 1.0f / sqrtf(ss / (float)HD + 1e-6f);
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const float w8[8] = {wq[c][0].x, wq[c][0].y, wq[c][0].z, wq[c][0].w,
                                     wq[c][1].x, wq[c][1].y, wq[c][1].z, wq[c][1].w};
#pragma unroll
                for (int e = 0; e < 8; e++) x[c][e] = x[c][e] * inv * w8[e];
            }
            const float cs[16] = {cs4[0].x, cs4[0].y, cs4[0].z, cs4[0].w, cs4[1].x, cs4[1].y, cs4[1].z, cs4[1].w,
                                  cs4[2].x, cs4[2].y, cs4[2].z, cs4[2].w, cs4[3].x, cs4[3].y, cs4[3].z, cs4[3].w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float c = cs[2 * e], sn = cs[2 * e + 1], a = x[0][e], bb = x[1][e];
                const float lo = rot ? a * c - bb * sn : a, hi = rot ? bb * c + a * sn : bb;
                q8[0][e] = (f16)((float)(f16)lo * scale);
                q8[1][e] = (f16)((float)(f16)hi * scale);
            }
        }
        *reinterpret_cast<f16x8*>(&Qs[qq][8 * c0]) = q8[0];
        *reinterpret_cast<f16x8*>(&Qs[qq][8 * c1]) = q8[1];
    }
    __syncthreads();
#pragma unroll
    for (int st = 0; st < NS; st++) qf[st] = *reinterpret_cast<const f16x8*>(&Qs[fq][st * 32 + fg * 8]);
    while (j < kend) {
        int jn = next_block(j + 4 * KB);
        process(j, kA, vA, jn, kB, vB);
        j = jn;
        if (j >= kend) break;
        jn = next_block(j + 4 * KB);
        process(j, kB, vB, jn, kA, vA);
        j = jn;
    }
    // merge the 4 waves: acc[dt][r] is O[query fq][dim 16dt + 4fg + r]
#pragma unroll
    for (int dt = 0; dt < ND; dt++)
#pragma unroll
        for (int r = 0; r < 4; r++) Om[wv][fq][dt * 16 + fg * 4 + r] = acc[dt][r];
    if (fg == 0) {
        Mm[wv][fq] = m_run;
        Lm[wv][fq] = l_run;
    }
    __syncthreads();
    // per query (thread q): the merged max, the weight of each wave's state, the merged sum
    __shared__ float Fw[16][4], Ml[16][2];
    if (tid < nq) {
        const int q = tid;
        float m = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++)
            if (Lm[w][q] > 0.f) m = fmaxf(m, Mm[w][q]);
        float l = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float f = Lm[w][q] > 0.f ? exp2_fast(Mm[w][q] - m) : 0.f;
            l += Lm[w][q] * f;
            Fw[q][w] = f;
        }
        Ml[q][0] = m;
        Ml[q][1] = l;
    }
    __syncthreads();
    // Thread (qe, d0): the 4 waves' partial outputs of query qe at dimensions d0 .. d0 + 15, summed
    // in wave order (16-byte LDS reads), then 16-byte stores.  Every LDS read comes first (a store
    // through a generic pointer keeps the compiler from moving LDS reads past it).
    float av[16];
#pragma unroll
    for (int u = 0; u < 16; u++) av[u] = 0.f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const float f = Fw[qe][w];
#pragma unroll
        for (int u4 = 0; u4 < 4; u4++) {
            const float4 v = *reinterpret_cast<const float4*>(&Om[w][qe][d0 + 4 * u4]);
            av[4 * u4] += v.x * f;
            av[4 * u4 + 1] += v.y * f;
            av[4 * u4 + 2] += v.z * f;
            av[4 * u4 + 3] += v.w * f;
        }
    }
    const float mq = Ml[qe][0], lq = Ml[qe][1];
    if (qe >= nq) return;
    const int t = t0 + qe;
    if (ks == 1) {
        // out = acc / l * sigmoid(gate), the sigmoid on the hardware exp2 and reciprocal (within about
        // 1 ulp in f32, rounded to f16)
        const float inv_l = 1.0f / lq;
        f16x8 o8[2];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const float g = (float)gv[u >> 3][u & 7];
            const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -LOG2E));
            o8[u >> 3][u & 7] = (f16)(av[u] * inv_l * sg);
        }
        f16* op = out + (size_t)t * s.HQ * HD + h * HD + d0;
        *reinterpret_cast<f16x8*>(op) = o8[0];
        *reinterpret_cast<f16x8*>(op + 8) = o8[1];
    } else {
        const size_t r = ((size_t)z * L + t) * s.HQ + h;
        float4* pp = reinterpret_cast<float4*>(pacc + r * HD + d0);
#pragma unroll
        for (int u4 = 0; u4 < 4; u4++) pp[u4] = float4{av[4 * u4], av[4 * u4 + 1], av[4 * u4 + 2], av[4 * u4 + 3]};
        if (d0 == 0) {
            pml[r * 2] = mq;
            pml[r * 2 + 1] = lq;
        }
    }
}

template <int HD>
__global__ __launch_bounds__(HD) void k_attn_combine(const float* __restrict__ pacc, const float* __restrict__ pml,
                                                     const f16* __restrict__ big, f16* __restrict__ out, int L, int ks,
                                                     int HQ, int stride) {
    const AttnShape s{HQ, 0, HD, 0, stride, 0};
    const int t = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
    // Every load is issued up front and unconditionally (splits past ks re-read the last one and are
    // then skipped), so none waits behind a branch or another load; the sums run in split order.
    float mz[ATTN_KS_MAX], lz[ATTN_KS_MAX], az[ATTN_KS_MAX];
#pragma unroll
    for (int z = 0; z < ATTN_KS_MAX; z++) {
        const size_t r = ((size_t)min(z, ks - 1) * L + t) * s.HQ + h;
        mz[z] = pml[r * 2];
        lz[z] = pml[r * 2 + 1];
        az[z] = pacc[r * HD + d];
    }
    const float g = (float)big[(size_t)t * s.stride + h * 2 * HD + HD + d];
    float m = -INFINITY;
#pragma unroll
    for (int z = 0; z < ATTN_KS_MAX; z++)
        if (z < ks && lz[z] > 0.f) m = fmaxf(m, mz[z]);
    float l = 0.f, a = 0.f;
#pragma unroll
    for (int z = 0; z < ATTN_KS_MAX; z++)
        if (z < ks && lz[z] > 0.f) {
            const float f = exp2_fast(mz[z] - m);
            l += lz[z] * f;
            a += az[z] * f;
        }
    // as k_attn's unsplit epilogue: acc / l * sigmoid(gate), the sigmoid on exp2 and the reciprocal
    out[(size_t)t * s.HQ * HD + h * HD + d] =
        (f16)(a * (1.0f / l) * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -LOG2E)));
}

}  // namespace

void qk_prep(const f16* big, const AttnShape& s, const float* qw, const float* kw, const float* rope, int L,
             const uint32_t* lu, const Segs& sg, f16* Q, f16* Kc, f16* Vc, hipStream_t st) {
    SD_CHECK(s.HD == 256, "attention: only head_dim 256 is supported");
    SD_CHECK(s.RD % 2 == 0 && s.RD <= s.HD, "attention: bad rotary_dim");
    SD_CHECK(s.stride % 4 == 0, "attention: the row stride must be a multiple of 4");
    SD_CHECK(s.ctx % 32 == 0, "attention: the cache length must be a multiple of 32");
    hipLaunchKernelGGL(k_qk_prep<256>, dim3((L + 3) / 4, Q ? s.HQ + s.HK : s.HK), dim3(256), 0, st, big, lu, L, s.HQ,
                       s.HK, s.RD, s.stride, s.ctx, sg.row, qw, kw, rope, Q, Kc, Vc);
    launched("qk_prep");
}

// Workspace (floats) the key-split path needs for up to `rows` query rows.
size_t attn_ws_floats(int rows, const AttnShape& s) { return (size_t)ATTN_KS_MAX * rows * s.HQ * (s.HD + 2); }

void attention_split(const f16* Q, const f16* Kc, const f16* Vc, const f16* big, const AttnShape& s, int L,
                     const uint32_t* lu, const Segs& sg, int ks, float* ws, f16* out, hipStream_t st, const float* qw,
                     const float* rope) {
    SD_CHECK(s.HD == 256 && s.HQ % s.HK == 0, "attention: unsupported head shape");
    SD_CHECK(Q || (qw && rope && s.RD == 64), "attention: the fused query norm and RoPE take rotary_dim 64");
    SD_CHECK(ks >= 1 && ks <= ATTN_KS_MAX, "attention: 1 to 8 key splits");
    const int nb = (L + BQ - 1) / BQ;
    float* pacc = ws;
    float* pml = ws + (size_t)ks * L * s.HQ * s.HD;
    if (Q)
        hipLaunchKernelGGL((k_attn<256, 0>), dim3(nb, s.HQ, ks), dim3(256), 0, st, Q, Kc, Vc, lu, L, s.HQ, s.HK, s.stride,
                           s.ctx, ks, sg.row, big, out, pacc, pml, qw, rope, s.RD);
    else
        hipLaunchKernelGGL((k_attn<256, 64>), dim3(nb, s.HQ, ks), dim3(256), 0, st, Q, Kc, Vc, lu, L, s.HQ, s.HK, s.stride,
                           s.ctx, ks, sg.row, big, out, pacc, pml, qw, rope, s.RD);
    launched("attn");
    if (ks > 1) {
        hipLaunchKernelGGL(k_attn_combine<256>, dim3(L, s.HQ), dim3(256), 0, st, pacc, pml, big, out, L, ks, s.HQ,
                           s.stride);
        launched("attn_combine");
    }
}

}  // namespace sd
