// Fused-dequant int4 (group 32, symmetric) GEMM on gfx950 MFMA:
//   Y[M,N] f16 = A[M,K] f16 . deq(W[N,K])^T, f32 accumulation.
// The reference's matmul kernels are src/kernels.rs:590-709 (GEMV with f32 dequant for M <= 20,
// tiled with f16 dequant otherwise; selection at src/engine.rs:414-444).
//
// Design (one kernel family for prefill and the short question suffix):
//  * a workgroup is 4 waves side by side along N; each wave owns NT 16-column tiles and all MT
//    16-row tiles of the workgroup, so no two waves ever dequantize the same weights;
//  * weights go straight from HBM to registers: lane (j = l%16, g = l/16) loads the whole 16-byte
//    quant block (32 k values) of column j at block kb0+g, i.e. one macro step covers 128 k and
//    feeds 4 v_mfma_f32_16x16x32_f16; step s uses word s of the block;
//  * a word's 8 nibbles become 4 f16 pairs with the 0x6400 exponent trick:
//      (w & 0x000F000F) | 0x64006400 = (1024 + q0, 1024 + q4), minus 1032 (exact) gives q - 8;
//      (w & 0x00F000F0) | 0x64006400 = (1024 + 16 q1, 1024 + 16 q5), times 1/16 minus 72 (one
//      exact fma) gives q - 8; the same on w >> 8 gives q2/q6 and q3/q7.  Times the f16 scale
//    rounds once: exactly the reference's f16 dequant (f16(q) - 8) * sc.  The pairs come out in
//    k order [0,4,1,5,2,6,3,7]; the A tile is stored to LDS in the same order, so the dot
//    products see matching k;
//  * `EXACT` reproduces the reference GEMV's f32 dequant (q-8)*sc: the value is split into
//    hi = f16((q-8)*sc) and lo = fma_f16(q-8, sc, -hi) (exact: the residual is a multiple of
//    2^-24 with at most 5 significant bits), and both are fed to the MFMA;
//  * A (activations, f16) is staged once per workgroup per macro step in a double-buffered LDS
//    tile shared by the 4 waves (one barrier per step), with A two steps and B one step ahead in
//    registers;
//  * split-K over workgroups writes f32 partials [ks][M][N] with plain stores and no cross-
//    workgroup synchronisation (on MI355X a device-scope fence writes back the whole XCD L2); the
//    consumer sums the ks slots in a fixed order: the residual add + RMSNorm does it for the
//    projections that feed it, `reduce_partials` for everything else.
#include "common.h"

namespace sd {
namespace {

constexpr int KSTEP = 128;      // k per macro step: 4 quant blocks
#ifndef SD_LDA_PAD
#define SD_LDA_PAD 8
#endif
constexpr int LDA = KSTEP + SD_LDA_PAD;  // LDS row stride in halves

// The 8 nibbles of a weight word as 4 f16 pairs q - 8 (exact), k order [0,4],[1,5],[2,6],[3,7]:
// the low nibble of each byte lands in the f16 mantissa as 1024 + q, the high nibble as
// 1024 + 16 q, so two masks per 8-bit shift give all four pairs.
// (a & m) | c in one v_and_or_b32 (the compiler otherwise emits separate and/or here).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "s"(c));
    return r;
}

__device__ __forceinline__ void nib_pairs(uint32_t w, f16x2& p0, f16x2& p1, f16x2& p2, f16x2& p3) {
    const uint32_t w8 = w >> 8;
    const f16x2 x0 = __builtin_bit_cast(f16x2, and_or(w, 0x000F000Fu, 0x64006400u));
    const f16x2 x1 = __builtin_bit_cast(f16x2, and_or(w, 0x00F000F0u, 0x64006400u));
    const f16x2 x2 = __builtin_bit_cast(f16x2, and_or(w8, 0x000F000Fu, 0x64006400u));
    const f16x2 x3 = __builtin_bit_cast(f16x2, and_or(w8, 0x00F000F0u, 0x64006400u));
    const f16x2 c1032 = {(f16)1032.0f, (f16)1032.0f}, c16 = {(f16)0.0625f, (f16)0.0625f}, c72 = {(f16)-72.0f, (f16)-72.0f};
    p0 = x0 - c1032;
    p1 = __builtin_elementwise_fma(x1, c16, c72);
    p2 = x2 - c1032;
    p3 = __builtin_elementwise_fma(x3, c16, c72);
}

__device__ __forceinline__ f16x8 cat4(f16x2 a, f16x2 b, f16x2 c, f16x2 d) {
    return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Permute 8 halves [a0..a7] (as 4 words) to [a0,a4,a1,a5,a2,a6,a3,a7].
__device__ __forceinline__ u32x4 perm_a(u32x4 d) {
    u32x4 o;  // v_perm_b32: selector bytes 0-3 pick from the second source, 4-7 from the first
    o[0] = __builtin_amdgcn_perm(d[2], d[0], 0x05040100u);
    o[1] = __builtin_amdgcn_perm(d[2], d[0], 0x07060302u);
    o[2] = __builtin_amdgcn_perm(d[3], d[1], 0x05040100u);
    o[3] = __builtin_amdgcn_perm(d[3], d[1], 0x07060302u);
    return o;
}

template <int MT, int NT, bool EXACT, bool PARTIAL>
__global__ __launch_bounds__(256) void k_gemm_w4(const f16* __restrict__ A, const uint32_t* __restrict__ W,
                                                 const f16* __restrict__ S, f16* __restrict__ Y,
                                                 float* __restrict__ part, int M, int N, int K, int ksplit) {
    constexpr int BM = MT * 16;
    constexpr int BN = 4 * NT * 16;
    constexpr int ACH = BM * 16 / 256;  // 16-byte A chunks per thread per macro step (== MT)
    // Double-buffered A tile: two separate arrays so that the compiler can see that the stores of
    // the next tile never alias the fragment reads of the current one.
    __shared__ __attribute__((aligned(16))) f16 As0[BM * LDA];
    __shared__ __attribute__((aligned(16))) f16 As1[BM * LDA];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, g = lane >> 4;
    // XCD-aware tile order: workgroup b runs on XCD b % 8, so XCD x is given the contiguous run of
    // tiles [x G/8, (x+1) G/8) in column-block-major order (every row block and K split of a column
    // block together): a column block's weights are then fetched into one XCD's L2 only.
    const int gy = gridDim.y, gyz = gridDim.y * gridDim.z;
    const int G = gridDim.x * gyz;
    const int b = blockIdx.x + gridDim.x * (blockIdx.y + gy * blockIdx.z);
    const int q8 = G >> 3;
    const int tile = b < 8 * q8 ? (b & 7) * q8 + (b >> 3) : b;
    const int bx = tile / gyz, by = (tile % gyz) % gy, bz = (tile % gyz) / gy;
    const int m0 = by * BM, n0 = bx * BN;
    const int KB = K >> 5;
    const int steps_total = K / KSTEP;
    const int steps = steps_total / ksplit;
    const int step0 = bz * steps;

    int ncol[NT];
    bool nok[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        ncol[t] = n0 + (wave * NT + t) * 16 + j;
        nok[t] = ncol[t] < N;
    }
    // Loads are branch-free: rows past M and columns past N read the last valid row/column, and
    // the outputs they feed are never stored.
    const u32x4* wrow[NT];
    const f16* srow[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const size_t n = (size_t)min(ncol[t], N - 1);
        wrow[t] = reinterpret_cast<const u32x4*>(W) + n * KB + g;
        srow[t] = S + n * KB + g;
    }
    const f16* arow[ACH];
#pragma unroll
    for (int c = 0; c < ACH; c++) {
        const int idx = tid + 256 * c;
        arow[c] = A + (size_t)min(m0 + (idx >> 4), M - 1) * K + (idx & 15) * 8;
    }

    f32x4 acc[MT][NT];
#pragma unroll
    for (int a = 0; a < MT; a++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[a][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 areg[ACH], bcur[NT], bnext[NT];
    f16 scur[NT], snext[NT];
    auto load_a = [&](int step) {
#pragma unroll
        for (int c = 0; c < ACH; c++) areg[c] = *reinterpret_cast<const u32x4*>(arow[c] + step * KSTEP);
    };
    auto load_b = [&](int step) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            bnext[t] = wrow[t][step * 4];
            snext[t] = srow[t][step * 4];
        }
    };
    auto store_a = [&](f16* dst) {
#pragma unroll
        for (int c = 0; c < ACH; c++) {
            const int idx = tid + 256 * c;
            *reinterpret_cast<u32x4*>(&dst[(idx >> 4) * LDA + (idx & 15) * 8]) = perm_a(areg[c]);
        }
    };
    auto frags = [&](const f16* Acur, int s, f16x8* af) {
#pragma unroll
        for (int a = 0; a < MT; a++)
            af[a] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(&Acur[(a * 16 + j) * LDA + g * 32 + s * 8]));
    };
    auto dequant = [&](int s, f16x8* b, f16x8* blo) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const f16x2 sc2 = f16x2{scur[t], scur[t]};
            f16x2 p0, p1, p2, p3;
            nib_pairs(bcur[t][s], p0, p1, p2, p3);
            const f16x2 h0 = p0 * sc2, h1 = p1 * sc2, h2 = p2 * sc2, h3 = p3 * sc2;
            b[t] = cat4(h0, h1, h2, h3);
            if constexpr (EXACT)
                blo[t] = cat4(__builtin_elementwise_fma(p0, sc2, -h0), __builtin_elementwise_fma(p1, sc2, -h1),
                              __builtin_elementwise_fma(p2, sc2, -h2), __builtin_elementwise_fma(p3, sc2, -h3));
        }
    };
    // One k step (4 sub-steps of 32 k).  The next tile's A store and the next loads are issued
    // first; sub-step s+1's fragment reads and dequant are issued before sub-step s's MFMAs.
    auto step = [&](const f16* Acur, f16* Anext, int it) {
        f16x8 af[2][MT], bf[2][NT], bl[2][EXACT ? NT : 1];
        frags(Acur, 0, af[0]);
        dequant(0, bf[0], bl[0]);
        if (it + 1 < steps) {
            store_a(Anext);
            load_b(step0 + it + 1);
            if (it + 2 < steps) load_a(step0 + it + 2);
        }
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int cu = s & 1, nx = cu ^ 1;
            if (s < 3) {
                frags(Acur, s + 1, af[nx]);
                dequant(s + 1, bf[nx], bl[nx]);
            }
#pragma unroll
            for (int a = 0; a < MT; a++)
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    acc[a][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[cu][a], bf[cu][t], acc[a][t], 0, 0, 0);
                    if constexpr (EXACT)
                        acc[a][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[cu][a], bl[cu][t], acc[a][t], 0, 0, 0);
                }
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            bcur[t] = bnext[t];
            scur[t] = snext[t];
        }
        __syncthreads();  // Anext is complete and Acur is no longer read
    };

    load_a(step0);
    load_b(step0);
#pragma unroll
    for (int t = 0; t < NT; t++) {
        bcur[t] = bnext[t];
        scur[t] = snext[t];
    }
    store_a(As0);
    if (steps > 1) load_a(step0 + 1);
    __syncthreads();
    for (int it = 0; it < steps; it += 2) {
        step(As0, As1, it);
        if (it + 1 < steps) step(As1, As0, it + 1);
    }

    // Output: acc[a][t][r] is row m0 + 16a + 4g + r, column ncol[t].
    if constexpr (!PARTIAL) {
#pragma unroll
        for (int a = 0; a < MT; a++)
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = m0 + a * 16 + g * 4 + r;
                    if (m < M && nok[t]) Y[(size_t)m * N + ncol[t]] = (f16)acc[a][t][r];
                }
        return;
    }
    float* mine = part + (size_t)bz * M * N;
#pragma unroll
    for (int a = 0; a < MT; a++)
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + a * 16 + g * 4 + r;
                if (m < M && nok[t]) mine[(size_t)m * N + ncol[t]] = acc[a][t][r];
            }
}

// The same product on v_mfma_f32_32x32x16_f16, which on MI355X runs at twice the rate of the
// 16x16x32 form (measured: about 2.1 vs 1.2 PFLOP/s).  Prefill only (f16 dequant).
//  * a wave owns MT2 32-row tiles x NT2 32-column tiles; 4 waves side by side along N;
//  * lane (r = l%32, g = l/32) holds column r of a column tile and dequantizes quant blocks 2g and
//    2g+1 of each 128-wide k step; MFMA k-slice s (16 k) takes word s%4 of block 2g + s/4 in lane
//    group g, so the A fragment of lane (r, g) is the 8 halves of row r at
//    k = 64g + 32(s/4) + 8(s%4) (the A tile sits in LDS in the nibble pair order, as above);
//  * D of the 32x32 tile: register i of lane l is row 8(i/4) + 4(l/32) + i%4, column l%32.
template <int MT2, int NT2, bool PARTIAL>
__global__ __launch_bounds__(256) void k_gemm_w4x(const f16* __restrict__ A, const uint32_t* __restrict__ W,
                                                  const f16* __restrict__ S, f16* __restrict__ Y,
                                                  float* __restrict__ part, int M, int N, int K, int ksplit) {
    constexpr int BM = MT2 * 32;
    constexpr int BN = 4 * NT2 * 32;
    constexpr int ACH = BM * 16 / 256;  // 16-byte A chunks per thread per k step
    __shared__ __attribute__((aligned(16))) f16 As0[BM * LDA];
    __shared__ __attribute__((aligned(16))) f16 As1[BM * LDA];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 31, g = lane >> 5;
    // XCD-aware tile order, as in k_gemm_w4
    const int gy = gridDim.y, gyz = gridDim.y * gridDim.z;
    const int G = gridDim.x * gyz;
    const int b = blockIdx.x + gridDim.x * (blockIdx.y + gy * blockIdx.z);
    const int q8 = G >> 3;
    const int tile = b < 8 * q8 ? (b & 7) * q8 + (b >> 3) : b;
    const int bx = tile / gyz, by = (tile % gyz) % gy, bz = (tile % gyz) / gy;
    const int m0 = by * BM, n0 = bx * BN;
    const int KB = K >> 5;
    const int steps = (K / KSTEP) / ksplit;
    const int step0 = bz * steps;

    int ncol[NT2];
    const u32x4* wrow[NT2];
    const f16* srow[NT2];
#pragma unroll
    for (int t = 0; t < NT2; t++) {
        ncol[t] = n0 + (wave * NT2 + t) * 32 + r;
        const size_t n = (size_t)min(ncol[t], N - 1);
        wrow[t] = reinterpret_cast<const u32x4*>(W) + n * KB + 2 * g;
        srow[t] = S + n * KB + 2 * g;
    }
    const f16* arow[ACH];
#pragma unroll
    for (int c = 0; c < ACH; c++) {
        const int idx = tid + 256 * c;
        arow[c] = A + (size_t)min(m0 + (idx >> 4), M - 1) * K + (idx & 15) * 8;
    }

    f32x16 acc[MT2][NT2];
#pragma unroll
    for (int a = 0; a < MT2; a++)
#pragma unroll
        for (int t = 0; t < NT2; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[a][t][i] = 0.f;

    u32x4 areg[ACH], bcur[NT2][2], bnext[NT2][2];
    f16 scur[NT2][2], snext[NT2][2];
    auto load_a = [&](int step) {
#pragma unroll
        for (int c = 0; c < ACH; c++) areg[c] = *reinterpret_cast<const u32x4*>(arow[c] + step * KSTEP);
    };
    auto load_b = [&](int step) {
#pragma unroll
        for (int t = 0; t < NT2; t++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                bnext[t][h] = wrow[t][step * 4 + h];
                snext[t][h] = srow[t][step * 4 + h];
            }
    };
    auto store_a = [&](f16* dst) {
#pragma unroll
        for (int c = 0; c < ACH; c++) {
            const int idx = tid + 256 * c;
            *reinterpret_cast<u32x4*>(&dst[(idx >> 4) * LDA + (idx & 15) * 8]) = perm_a(areg[c]);
        }
    };
    auto frags = [&](const f16* Acur, int s, f16x8* af) {
#pragma unroll
        for (int a = 0; a < MT2; a++)
            af[a] = __builtin_bit_cast(
                f16x8, *reinterpret_cast<const u32x4*>(&Acur[(a * 32 + r) * LDA + 64 * g + 32 * (s >> 2) + 8 * (s & 3)]));
    };
    auto dequant = [&](int s, f16x8* bf) {
#pragma unroll
        for (int t = 0; t < NT2; t++) {
            const f16 sc = scur[t][s >> 2];
            const f16x2 sc2 = f16x2{sc, sc};
            f16x2 p0, p1, p2, p3;
            nib_pairs(bcur[t][s >> 2][s & 3], p0, p1, p2, p3);
            bf[t] = cat4(p0 * sc2, p1 * sc2, p2 * sc2, p3 * sc2);
        }
    };
    // One k step = 8 MFMA k-slices; slice s+1's fragments and dequant are issued before slice s's
    // MFMAs, the next tile's A store and loads first.
    auto step = [&](const f16* Acur, f16* Anext, int it) {
        f16x8 af[2][MT2], bf[2][NT2];
        frags(Acur, 0, af[0]);
        dequant(0, bf[0]);
        if (it + 1 < steps) {
            store_a(Anext);
            load_b(step0 + it + 1);
            if (it + 2 < steps) load_a(step0 + it + 2);
        }
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const int cu = s & 1, nx = cu ^ 1;
            if (s < 7) {
                frags(Acur, s + 1, af[nx]);
                dequant(s + 1, bf[nx]);
            }
#pragma unroll
            for (int a = 0; a < MT2; a++)
#pragma unroll
                for (int t = 0; t < NT2; t++)
                    acc[a][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cu][a], bf[cu][t], acc[a][t], 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < NT2; t++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                bcur[t][h] = bnext[t][h];
                scur[t][h] = snext[t][h];
            }
        __syncthreads();
    };

    load_a(step0);
    load_b(step0);
#pragma unroll
    for (int t = 0; t < NT2; t++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            bcur[t][h] = bnext[t][h];
            scur[t][h] = snext[t][h];
        }
    store_a(As0);
    if (steps > 1) load_a(step0 + 1);
    __syncthreads();
    for (int it = 0; it < steps; it += 2) {
        step(As0, As1, it);
        if (it + 1 < steps) step(As1, As0, it + 1);
    }

    float* mine = PARTIAL ? part + (size_t)bz * M * N : nullptr;
#pragma unroll
    for (int a = 0; a < MT2; a++)
#pragma unroll
        for (int t = 0; t < NT2; t++) {
            if (ncol[t] >= N) continue;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int m = m0 + a * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
                if (m >= M) continue;
                if constexpr (PARTIAL) mine[(size_t)m * N + ncol[t]] = acc[a][t][i];
                else Y[(size_t)m * N + ncol[t]] = (f16)acc[a][t][i];
            }
        }
}

// Y[i] = f16(sum_z part[z][i]) in slot order.
__global__ void k_reduce_partials(const float* __restrict__ part, int ks, size_t n, f16* __restrict__ Y) {
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= n) return;
    if (i + 4 <= n && (n & 3) == 0) {
        float4 s = *reinterpret_cast<const float4*>(part + i);
        for (int z = 1; z < ks; z++) {
            const float4 v = *reinterpret_cast<const float4*>(part + (size_t)z * n + i);
            s.x += v.x, s.y += v.y, s.z += v.z, s.w += v.w;
        }
        *reinterpret_cast<f16x4*>(Y + i) = f16x4{(f16)s.x, (f16)s.y, (f16)s.z, (f16)s.w};
        return;
    }
    for (size_t e = i; e < n && e < i + 4; e++) {
        float s = part[e];
        for (int z = 1; z < ks; z++) s += part[(size_t)z * n + e];
        Y[e] = (f16)s;
    }
}

typedef void (*GemmFn)(const f16*, const uint32_t*, const f16*, f16*, float*, int, int, int, int);
struct Cfg {
    int mt, nt;
    bool exact;
    GemmFn f16_out, part_out;
};

#define SD_CFG(MT, NT, EX) Cfg{MT, NT, EX, k_gemm_w4<MT, NT, EX, false>, k_gemm_w4<MT, NT, EX, true>}
#define SD_CFGX(MT2, NT2) Cfg{2 * MT2, 2 * NT2, false, k_gemm_w4x<MT2, NT2, false>, k_gemm_w4x<MT2, NT2, true>}
const Cfg kCfgs[] = {
    SD_CFG(1, 1, true), SD_CFG(2, 1, true),                                           // M <= 20: f32 dequant
    SD_CFG(1, 1, false), SD_CFG(2, 1, false), SD_CFG(3, 1, false), SD_CFG(4, 1, false),  // skinny
    SD_CFG(8, 2, false), SD_CFG(8, 4, false), SD_CFG(4, 2, false), SD_CFG(8, 1, false),  // prefill
    SD_CFG(4, 4, false), SD_CFG(6, 2, false), SD_CFG(3, 2, false), SD_CFG(2, 2, false),
    SD_CFG(4, 3, false), SD_CFG(3, 3, false), SD_CFG(2, 3, false), SD_CFG(5, 2, false),
    // 32x32x16 MFMA tiles (MT2 x 32 rows, 4 x NT2 x 32 columns), listed in 16-row / 64-column units
    SD_CFGX(2, 1), SD_CFGX(2, 2), SD_CFGX(4, 1), SD_CFGX(3, 1), SD_CFGX(1, 1), SD_CFGX(1, 2),
};
#undef SD_CFG
#undef SD_CFGX
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

int pick_cfg(int M, bool exact) {
    if (exact) return M <= 16 ? 0 : 1;
    if (M <= 16) return 2;
    if (M <= 32) return 3;
    if (M <= 48) return 4;
    if (M <= 64) return 5;
    return 8;  // (4, 2): the best prefill tile on MI355X in a sweep over the 2B's shapes
}

}  // namespace

int gemm_w4_configs() { return kNumCfgs; }

int gemm_w4_cfg(int M, bool exact) { return pick_cfg(M, exact); }

GemmPlan gemm_w4_plan(int M, int N, int K, bool exact, bool partial_ok, size_t max_part_elems) {
    GemmPlan p{pick_cfg(M, exact), 1};
    if (!exact && M >= 256 && M <= 1024) {
        // Prefill-sized M.  From a sweep of the 2B's shapes at M = 512 on MI355X (256 CUs, two
        // 256-thread workgroups each): filling whole rounds of workgroup slots matters more than a
        // tile's own speed, so the tile follows N.
        if (N >= 10000) p.cfg = 14;      // (4,3): N = 12288 -> 64 column blocks x 8 row blocks = 512
        else if (N >= 7000) p.cfg = 17;  // (5,2): N = 8256 -> 65 x 7 = 455
        else if (N >= 4000) p.cfg = 21;  // 32x32 (3,1): N = 5120 -> 40 x 6 = 240
        else if (partial_ok) {           // N = 2048: split K so that the grid covers the chip
            p.cfg = 18;                  // 32x32 (2,1): 16 x 8 tiles, x 4 splits (K = 6144) or x 2
            p.ks = K > 3000 ? 4 : 2;
        }
        const int steps = K / KSTEP;
        while (p.ks > 1 && (steps % p.ks || (size_t)p.ks * M * N > max_part_elems)) p.ks /= 2;
        return p;
    }
    if (!exact && M > 64 && M < 256) {
        // Batched questions and short prefills: 16-column tiles per wave stream the weights with
        // more workgroups in flight ((4,1) with split K where partials are allowed, else (3,1)).
        p.cfg = partial_ok ? 5 : 4;
    }
    if (partial_ok) p.ks = gemm_w4_split(M, N, K, p.cfg, 512, max_part_elems);
    return p;
}

int gemm_w4_split(int M, int N, int K, int cfg, int target_groups, size_t max_part_elems) {
    const Cfg& c = kCfgs[cfg];
    const int bm = c.mt * 16, bn = 4 * c.nt * 16;
    const int groups = ((N + bn - 1) / bn) * ((M + bm - 1) / bm);
    const int steps = K / KSTEP;
    int ks = 1;
    while (groups * ks < target_groups && ks < 8 && steps % (ks * 2) == 0 && steps / (ks * 2) >= 2 &&
           (size_t)(ks * 2) * M * N <= max_part_elems)
        ks *= 2;
    return ks;
}

void gemm_w4(const f16* A, const uint32_t* W, const f16* S, f16* Y, float* part, int M, int N, int K, bool exact,
             int ks, hipStream_t st, int cfg) {
    SD_CHECK(M >= 1 && N >= 1 && K >= KSTEP && K % KSTEP == 0, "gemm_w4: need M, N >= 1 and K a multiple of 128");
    const int ci = cfg >= 0 ? cfg : pick_cfg(M, exact);
    SD_CHECK(ci < kNumCfgs, "gemm_w4: bad configuration index");
    const Cfg& c = kCfgs[ci];
    SD_CHECK(c.exact == exact, "gemm_w4: configuration does not match the dequant mode");
    SD_CHECK(ks >= 1 && (K / KSTEP) % ks == 0, "gemm_w4: split count must divide the k steps");
    SD_CHECK(part || (Y && ks == 1), "gemm_w4: split-K writes partials and needs a partial buffer");
    const int bm = c.mt * 16, bn = 4 * c.nt * 16;
    dim3 grid((N + bn - 1) / bn, (M + bm - 1) / bm, ks);
    hipLaunchKernelGGL(part ? c.part_out : c.f16_out, grid, dim3(256), 0, st, A, W, S, Y, part, M, N, K, ks);
    launched("gemm_w4");
}

void reduce_partials(const float* part, int ks, size_t n, f16* Y, hipStream_t st) {
    const size_t threads = (n + 3) / 4;
    hipLaunchKernelGGL(k_reduce_partials, dim3((threads + 255) / 256), dim3(256), 0, st, part, ks, n, Y);
    launched("reduce_partials");
}

}  // namespace sd
