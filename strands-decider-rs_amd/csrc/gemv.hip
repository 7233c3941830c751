// Quantized GEMV on gfx950 MFMA: the reference's matmul_gemv (src/kernels.rs:590-635, decode
// 550-576), Y[M,N] = A[M,K] f16 . deq(W[N,K])^T with the weights dequantized in f32 and f32
// accumulation.  It serves the short question suffix (M <= 20, the reference's GEMV rows,
// src/engine.rs:419-425) and every matrix the tiled kernels do not take: non-default formats
// (int2/int3, asymmetric, group > 32) and N % 64 != 0 (src/engine.rs:434-442), at any M.
//
// Design (HBM/latency-bound weight streaming):
//  * v_mfma_f32_16x16x32_f16 with the weights as the row operand (16 output columns) and the
//    activations as the column operand (16 input rows): D[n][m].  The f32 dequantized value v is
//    split into hi = f16(v) and lo = f16(v - hi) and both go through the MFMA with the same
//    activations; for symmetric formats hi + lo is v exactly (the residual has at most 5 significant
//    bits), so the product is the reference's f32 dequant at f32 accumulation;
//  * a macro step is 128 k (4 quant blocks): lane (i = l % 16, g = l / 16) loads block g of column i
//    (16 bytes for int4) and the 64 bytes of input row i at those 32 k; MFMA k-slice q takes
//    element group q of both, so the operands need no permutation;
//  * a workgroup is 4 waves that split its k range (wave w takes macro steps w, w + 4, ...) and sum
//    their accumulators through LDS at the end, in a fixed order; every wave keeps 4 macro steps of
//    loads in flight (for K = 2048 that is all of them), with explicit vmcnt waits;
//  * workgroups split the columns in tiles of 16 x NCT; with f32 partial outputs the k range is also
//    split over ks workgroups (the consumer sums the slots in order, as for the tiled kernels);
//  * the gate_up of the short path (rows interleaved in groups of 16) can apply SiLU * mul in the
//    epilogue: a wave's two column tiles are then 16 gate and the 16 matching up columns;
//  * every load is a raw buffer load: columns past N, rows past M and k past K read zeros.
//
// Weight layouts: TILED is the engine's int4 group-32 layout (tile_w4, words in the engine nibble
// order of repack_w4); otherwise the reference's plain layout, [N][K/32] blocks of 4*bits bytes in
// the reference's bit order, scales (and asymmetric biases) [N][K/group] f16.
#include <hip/hip_ext.h>

#include "common.h"
#include "device.h"

namespace sd {
namespace {

constexpr int GV_PD = 4;  // macro steps (128 k) in flight per wave

template <int B>
struct BlkT;
template <>
struct BlkT<4> {
    typedef u32x4 T;
};
template <>
struct BlkT<3> {
    typedef u32x3 T;
};
template <>
struct BlkT<2> {
    typedef u32x2 T;
};

template <int B>
__device__ __forceinline__ typename BlkT<B>::T load_blk(Rsrc r, uint32_t off) {
    if constexpr (B == 4) return buf_b128(r, off, 0);
    else if constexpr (B == 3) return buf_b96(r, off, 0);
    else return buf_b64(r, off, 0);
}

// Elements 8q .. 8q + 7 of a quant block as f16 hi and lo parts of their f32 values.
// TILED: int4 in the engine nibble order (nib_pairs), v = (q - 8) sc with hi = f16 product and lo
// the exact residual (one f16 fma).  Plain: the reference's bit order (src/kernels.rs:550-576),
// v = (q - 2^(bits-1)) sc or fma(q, sc, bi) in f32.
template <int BITS, bool ASYM, bool TILED>
__device__ __forceinline__ void deq8(const typename BlkT<BITS>::T& w, uint32_t sc_bits, uint32_t bi_bits, int q,
                                     f16x8& hi, f16x8& lo) {
    const f16 sc = __builtin_bit_cast(f16, (uint16_t)sc_bits);
    if constexpr (TILED) {
        const f16x2 sc2 = f16x2{sc, sc};
        f16x2 p0, p1, p2, p3;
        nib_pairs(w[q], p0, p1, p2, p3);
        const f16x2 h0 = p0 * sc2, h1 = p1 * sc2, h2 = p2 * sc2, h3 = p3 * sc2;
        hi = cat4(h0, h1, h2, h3);
        lo = cat4(__builtin_elementwise_fma(p0, sc2, -h0), __builtin_elementwise_fma(p1, sc2, -h1),
                  __builtin_elementwise_fma(p2, sc2, -h2), __builtin_elementwise_fma(p3, sc2, -h3));
    } else {
        const float s = (float)sc;
        const float bi = ASYM ? (float)__builtin_bit_cast(f16, (uint16_t)bi_bits) : 0.f;
        uint32_t codes[8];
        if constexpr (BITS == 4) {
#pragma unroll
            for (int u = 0; u < 8; u++) codes[u] = (w[q] >> (4 * u)) & 15u;
        } else {
            const uint32_t lw = w[q >> 1] >> (16 * (q & 1));
#pragma unroll
            for (int u = 0; u < 8; u++) codes[u] = (lw >> (2 * u)) & 3u;
            if constexpr (BITS == 3) {
                const uint32_t hw = w[2] >> (8 * q);
#pragma unroll
                for (int u = 0; u < 8; u++) codes[u] |= ((hw >> u) & 1u) << 2;
            }
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float c = (float)codes[u];
            const float v = ASYM ? __builtin_fmaf(c, s, bi) : (c - (float)(1 << (BITS - 1))) * s;
            const f16 h = (f16)v;
            hi[u] = h;
            lo[u] = (f16)(v - (float)h);
        }
    }
}

// OUT: 0 = f16 Y [M][N]; 1 = f32 slot z of the split-K partials [ks][M][N]; 2 = f16 mid [M][N/2] =
// silu(gate) * up of gate_up rows interleaved in groups of 16 (NCT even: tile 2p is 16 gate columns,
// tile 2p + 1 the matching up columns), gate and up rounded to f16 first as the reference stores them.
template <int BITS, bool ASYM, bool TILED, int NCT, int MT, int OUT>
__global__ __launch_bounds__(256) void k_gemv(const f16* __restrict__ A, const uint32_t* __restrict__ W,
                                              const f16* __restrict__ S, const f16* __restrict__ Bi,
                                              void* __restrict__ Y, int M, int N, int K, int gdiv, int ks) {
    typedef typename BlkT<BITS>::T Blk;
    constexpr int BB = 4 * BITS;                            // bytes per quant block
    constexpr int LPS = NCT * (ASYM ? 3 : 2) + 4 * MT;      // loads a lane issues per macro step
    constexpr int WAIT = vmcnt_imm((GV_PD - 1) * LPS);      // all but the oldest step's loads
    static_assert((GV_PD - 1) * LPS <= 63, "vmcnt holds at most 63");
    static_assert(!TILED || (BITS == 4 && !ASYM), "the tiled layout is int4 group 32 symmetric");
    static_assert(OUT != 2 || NCT % 2 == 0, "SiLU pairs gate and up column tiles");
    __shared__ f32x4 red[4][NCT][MT][64];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * NCT * 16, m0 = blockIdx.y * MT * 16, z = blockIdx.z;
    const int KB = K >> 5, SM = (KB + 3) >> 2, SZ = (SM + ks - 1) / ks;
    const int sb = z * SZ, se = min(SM, sb + SZ);
    const int nst = se > sb + wave ? (se - sb - wave + 3) >> 2 : 0;  // this wave's steps: sb + wave + 4t
    const int KG = KB / gdiv;                                         // scale groups per column (plain)

    const Rsrc rw = make_rsrc(W, (uint32_t)N * KB * BB), rs = make_rsrc(S, (uint32_t)N * (TILED ? KB : KG) * 2),
               rb = make_rsrc(ASYM ? Bi : S, (uint32_t)N * KG * 2), ra = make_rsrc(A, (uint32_t)M * K * 2);

    Blk wr[GV_PD][NCT];
    uint32_t sr[GV_PD][NCT], br[GV_PD][NCT];
    u32x4 ar[GV_PD][MT][4];
    f32x4 acc[NCT][MT];
#pragma unroll
    for (int ct = 0; ct < NCT; ct++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[ct][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Loads of this wave's step t into ring slot `slot`: block b = 4 s + g of each column tile and
    // the matching 32 k of each input row (zeros past the wave's steps, N, M and K).
    auto issue = [&](int t, int slot) {
        const int b = 4 * (sb + wave + 4 * t) + g;
        const bool bok = t < nst && b < KB;
#pragma unroll
        for (int ct = 0; ct < NCT; ct++) {
            const int n = n0 + 16 * ct + i;
            uint32_t wo = OOB, so = OOB, bo = OOB;
            if (bok && n < N) {
                if constexpr (TILED) {
                    const uint32_t idx = ((uint32_t)(n >> 5) * (uint32_t)(KB >> 1) + (uint32_t)(b >> 1)) * 64u +
                                         (uint32_t)(n & 31) * 2u + (uint32_t)(b & 1);
                    wo = idx * 16u;
                    so = idx * 2u;
                } else {
                    wo = ((uint32_t)n * KB + b) * BB;
                    so = bo = ((uint32_t)n * KG + (uint32_t)(b / gdiv)) * 2u;
                }
            }
            wr[slot][ct] = load_blk<BITS>(rw, wo);
            sr[slot][ct] = buf_b16(rs, so, 0);
            if constexpr (ASYM) br[slot][ct] = buf_b16(rb, bo, 0);
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int m = m0 + 16 * mt + i;
            const uint32_t ao = bok && m < M ? ((uint32_t)m * K + 32u * b) * 2u : OOB;
#pragma unroll
            for (int q = 0; q < 4; q++) ar[slot][mt][q] = buf_b128(ra, ao + 16u * q, 0);
        }
        __builtin_amdgcn_sched_barrier(0);  // each step's loads stay together and in step order
    };
    auto compute = [&](int slot) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            f16x8 hi[NCT], lo[NCT];
#pragma unroll
            for (int ct = 0; ct < NCT; ct++)
                deq8<BITS, ASYM, TILED>(wr[slot][ct], sr[slot][ct], ASYM ? br[slot][ct] : 0u, q, hi[ct], lo[ct]);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const f16x8 av = __builtin_bit_cast(f16x8, ar[slot][mt][q]);
#pragma unroll
                for (int ct = 0; ct < NCT; ct++) {
                    acc[ct][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(hi[ct], av, acc[ct][mt], 0, 0, 0);
                    acc[ct][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(lo[ct], av, acc[ct][mt], 0, 0, 0);
                }
            }
        }
    };

    // Ring of GV_PD steps: wait for the oldest, use it, refill its slot with the step GV_PD later
    // (steps past this wave's count load nothing, so the wait counts stay exact).
    issue(0, 0);
    issue(1, 1);
    issue(2, 2);
    issue(3, 3);
    for (int t = 0; t < nst; t += GV_PD) {
        wait_loads<WAIT>();
        compute(0);
        issue(t + 4, 0);
        wait_loads<WAIT>();
        compute(1);
        issue(t + 5, 1);
        wait_loads<WAIT>();
        compute(2);
        issue(t + 6, 2);
        wait_loads<WAIT>();
        compute(3);
        issue(t + 7, 3);
    }
    wait_loads<vmcnt_imm(0)>();

    // The 4 waves' sums, added in wave order.  Lane l of tile (ct, mt) holds D[4 (l / 16) + r][l % 16]:
    // output column n0 + 16 ct + 4 (l / 16) + r of input row m0 + 16 mt + l % 16.
#pragma unroll
    for (int ct = 0; ct < NCT; ct++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) red[wave][ct][mt][lane] = acc[ct][mt];
    __syncthreads();
    auto total = [&](int ct, int mt, int l) {
        f32x4 v = red[0][ct][mt][l];
#pragma unroll
        for (int w = 1; w < 4; w++) {
            const f32x4 x = red[w][ct][mt][l];
            v[0] += x[0], v[1] += x[1], v[2] += x[2], v[3] += x[3];
        }
        return v;
    };
    if constexpr (OUT == 2) {
        f16* mid = static_cast<f16*>(Y);
        const int half = N >> 1;
        for (int it = tid; it < (NCT / 2) * MT * 64; it += 256) {
            const int l = it & 63, mt = (it >> 6) % MT, p = (it >> 6) / MT;
            const int m = m0 + 16 * mt + (l & 15);
            const int j = (n0 >> 1) + 16 * p + 4 * (l >> 4);
            if (m >= M || j >= half) continue;
            const f32x4 gv = total(2 * p, mt, l), uv = total(2 * p + 1, mt, l);
            f16x4 o;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float gg = (float)(f16)gv[r], uu = (float)(f16)uv[r];
                o[r] = (f16)silu_mul(gg, uu);
            }
            *reinterpret_cast<f16x4*>(mid + (size_t)m * half + j) = o;
        }
        return;
    }
    const bool vec = (N & 3) == 0;
    for (int it = tid; it < NCT * MT * 64; it += 256) {
        const int l = it & 63, mt = (it >> 6) % MT, ct = (it >> 6) / MT;
        const int m = m0 + 16 * mt + (l & 15), n = n0 + 16 * ct + 4 * (l >> 4);
        if (m >= M || n >= N) continue;
        const f32x4 v = total(ct, mt, l);
        if constexpr (OUT == 0) {
            f16* y = static_cast<f16*>(Y) + (size_t)m * N + n;
            if (vec) {
                *reinterpret_cast<f16x4*>(y) = f16x4{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (n + r < N) y[r] = (f16)v[r];
            }
        } else {
            float* y = static_cast<float*>(Y) + ((size_t)z * M + m) * N + n;
            if (vec) {
                __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(y));
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (n + r < N) y[r] = v[r];
            }
        }
    }
}

typedef void (*GemvFn)(const f16*, const uint32_t*, const f16*, const f16*, void*, int, int, int, int, int);

template <int BITS, bool ASYM, bool TILED, int NCT>
GemvFn pick_mt(int mt, int out) {
    if (mt == 1) {
        if (out == 0) return k_gemv<BITS, ASYM, TILED, NCT, 1, 0>;
        if (out == 1) return k_gemv<BITS, ASYM, TILED, NCT, 1, 1>;
        if constexpr (NCT % 2 == 0) return k_gemv<BITS, ASYM, TILED, NCT, 1, 2>;
    } else {
        if (out == 0) return k_gemv<BITS, ASYM, TILED, NCT, 2, 0>;
        if (out == 1) return k_gemv<BITS, ASYM, TILED, NCT, 2, 1>;
        if constexpr (NCT % 2 == 0) return k_gemv<BITS, ASYM, TILED, NCT, 2, 2>;
    }
    return nullptr;
}

GemvFn pick_gemv(int bits, bool asym, bool tiled, int nct, int mt, int out) {
    if (tiled) return nct == 2 ? pick_mt<4, false, true, 2>(mt, out) : pick_mt<4, false, true, 1>(mt, out);
    if (out == 2) return nullptr;
    switch (bits * 2 + (asym ? 1 : 0)) {
        case 8: return pick_mt<4, false, false, 1>(mt, out);
        case 9: return pick_mt<4, true, false, 1>(mt, out);
        case 6: return pick_mt<3, false, false, 1>(mt, out);
        case 7: return pick_mt<3, true, false, 1>(mt, out);
        case 4: return pick_mt<2, false, false, 1>(mt, out);
        case 5: return pick_mt<2, true, false, 1>(mt, out);
        default: return nullptr;
    }
}

}  // namespace

GemvPlan gemv_plan(int M, int N, int K, bool tiled, int out, size_t max_part_elems) {
    GemvPlan p;
    p.mt = M <= 16 ? 1 : 2;
    const int rb = (M + 16 * p.mt - 1) / (16 * p.mt);
    // f16 outputs own their whole k range; two column tiles per workgroup where that still gives
    // about one workgroup per CU (or more), one otherwise
    p.nct = tiled && (out == 2 || (size_t)((N + 31) / 32) * rb >= 240) ? 2 : 1;
    p.ks = 1;
    if (out == 1) {
        // partials: split k until the grid covers the chip (each wave keeps >= 1 macro step)
        const int groups = ((N + 16 * p.nct - 1) / (16 * p.nct)) * rb;
        const int SM = (K / 32 + 3) / 4;
        while (p.ks < 8 && groups * p.ks < 256 && SM / (p.ks * 2) >= 4 &&
               (size_t)(p.ks * 2) * M * N <= max_part_elems)
            p.ks *= 2;
    }
    return p;
}

void gemv(const f16* A, const uint32_t* W, const f16* S, const f16* Bi, void* Y, int out, int M, int N, int K, int bits,
          int group, bool asym, bool tiled, const GemvPlan& p, hipStream_t st) {
    SD_CHECK(M >= 1 && N >= 1 && K >= 32 && K % 32 == 0, "gemv: need M, N >= 1 and K a multiple of 32");
    SD_CHECK(bits == 2 || bits == 3 || bits == 4, "gemv: weights must be int2, int3 or int4");
    SD_CHECK(group >= 32 && group % 32 == 0 && K % group == 0, "gemv: the group must be a multiple of 32 dividing K");
    SD_CHECK(!tiled || (bits == 4 && group == 32 && !asym && w4_tileable(N, K)),
             "gemv: the tiled layout is int4 group 32 symmetric with N a multiple of 32");
    SD_CHECK(out != 2 || (tiled && p.nct == 2 && N % 32 == 0), "gemv: SiLU * mul needs the tiled gate_up in pairs");
    SD_CHECK(p.ks >= 1 && (out == 1 || p.ks == 1), "gemv: only partial outputs split k");
    SD_CHECK((size_t)N * (K / 32) * 4 * bits < 0x80000000u && (size_t)M * K * 2 < 0x80000000u,
             "gemv: operands must be below 2 GiB");
    const GemvFn f = pick_gemv(bits, asym, tiled, p.nct, p.mt, out);
    SD_CHECK(f, "gemv: no kernel for this format and output");
    const dim3 grid((N + 16 * p.nct - 1) / (16 * p.nct), (M + 16 * p.mt - 1) / (16 * p.mt), p.ks);
    const int gdiv = group / 32;
    KernelEvents* ke = kernel_events();
    if (ke && ke->launches == 0) {
        hipExtLaunchKernelGGL(f, grid, dim3(256), 0, st, ke->start, ke->stop, 0u, A, W, S, Bi, Y, M, N, K, gdiv, p.ks);
        ke->launches++;
    } else {
        hipLaunchKernelGGL(f, grid, dim3(256), 0, st, A, W, S, Bi, Y, M, N, K, gdiv, p.ks);
    }
    launched("gemv");
}

}  // namespace sd
