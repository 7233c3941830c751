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
//      (w & 0x000F000F) | 0x64006400 = (1024 + q, 1024 + q'), minus 1032 (exact) gives q - 8;
//      (w & 0x00F000F0) | 0x64006400 = (1024 + 16 q, 1024 + 16 q'), times 1/16 minus 72 (one
//      exact fma) gives q - 8; the same on w >> 8 gives the other two pairs.  Times the f16 scale
//    rounds once: exactly the reference's f16 dequant (f16(q) - 8) * sc.  The engine stores the
//    words in its own nibble order (k_repack_w4, run once at load), in which the four pairs are
//    (k0,k1), (k2,k3), (k4,k5), (k6,k7): the B fragments come out in natural k order and the A
//    tile needs no permutation;
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
//
// Weight layouts (both in the engine nibble order): `plain` is the model file's [N][K/32] blocks of
// 16 bytes with scales [N][K/32]; `tiled` (N % 32 == 0, K % 64 == 0, tile_w4 at load) stores each
// tile of 32 columns x 64 k (2 blocks per column) as one contiguous KiB, column-major inside:
// block (n, b) at 16-byte index ((n / 32) * (K / 64) + b / 2) * 64 + (n % 32) * 2 + b % 2, its scale
// at the same f16 index.  A wave's weights for one k step are then one KiB of whole cache lines
// (and 128 bytes of scales) instead of 16 or 2 bytes out of every column's lines.
#include <hip/hip_ext.h>

#include "common.h"
#include "device.h"

namespace sd {
namespace {

constexpr int KSTEP = 128;      // k per macro step: 4 quant blocks
#ifndef SD_LDA_PAD
#define SD_LDA_PAD 8
#endif
constexpr int LDA = KSTEP + SD_LDA_PAD;  // LDS row stride in halves

template <int MT, int NT, bool EXACT, bool PARTIAL>
__global__ __launch_bounds__(256) void k_gemm_w4(const f16* __restrict__ A, const uint32_t* __restrict__ W,
                                                 const f16* __restrict__ S, f16* __restrict__ Y,
                                                 float* __restrict__ part, int M, int N, int K, int ks_tiled) {
    constexpr int BM = MT * 16;
    constexpr int BN = 4 * NT * 16;
    const int ksplit = ks_tiled >> 1, tiled = ks_tiled & 1;
    constexpr int ACH = BM * 16 / 256;  // 16-byte A chunks per thread per macro step (== MT)
    // Double-buffered A tile: two separate arrays so that the compiler can see that the stores of
    // the next tile never alias the fragment reads of the current one.
    __shared__ __attribute__((aligned(16))) f16 As0[BM * LDA];
    __shared__ __attribute__((aligned(16))) f16 As1[BM * LDA];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, g = lane >> 4;
    int bx, by, bz;
    // the launch grid (ceil(N / BN), ceil(M / BM), ksplit) from the arguments, not from the dispatch
    // packet's grid size (one more scalar load before the first weight load could be issued)
    xcd_tile(blockIdx.x + (N + BN - 1) / BN * (blockIdx.y + (M + BM - 1) / BM * blockIdx.z), (N + BN - 1) / BN,
             (M + BM - 1) / BM, ksplit, bx, by, bz);
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
    // block kb0 + g of column n: plain n * KB + kb0 + g; tiled (kb0 a multiple of 4) the tile
    // step (kb0 + g) / 2 of column tile n / 32
    const u32x4* wrow[NT];
    const f16* srow[NT];
    const int wst = tiled ? 128 : 4;  // 16-byte blocks (and scales) per macro step of 128 k
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const size_t n = (size_t)min(ncol[t], N - 1);
        const size_t i0 = tiled ? ((n >> 5) * (size_t)(KB >> 1) + (g >> 1)) * 64 + (n & 31) * 2 + (g & 1) : n * KB + g;
        wrow[t] = reinterpret_cast<const u32x4*>(W) + i0;
        srow[t] = S + i0;
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
            bnext[t] = wrow[t][step * wst];
            snext[t] = srow[t][step * wst];
        }
    };
    auto store_a = [&](f16* dst) {
#pragma unroll
        for (int c = 0; c < ACH; c++) {
            const int idx = tid + 256 * c;
            *reinterpret_cast<u32x4*>(&dst[(idx >> 4) * LDA + (idx & 15) * 8]) = areg[c];
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
        lds_barrier();  // Anext is complete and Acur is no longer read (the loads ahead stay in flight)
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
    lds_barrier();
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

// The 16x16 product with the loads issued three k steps ahead (batched questions and other short M,
// where a workgroup's k chain is short and every step would otherwise wait for its weights):
//  * a workgroup is 4 waves side by side along N (NT 16-column tiles each) over MT 16-row tiles,
//    k in steps of 128 through a ring of 4 LDS stages, one barrier per step;
//  * the A tile of a step (BM rows x 256 B) goes straight from HBM to LDS (buffer_load_dwordx4 lds):
//    16-byte chunk q of the stage (q = (i * 4 + wave) * 64 + lane for the thread's i-th load) holds
//    row q / 16, k-chunk (q % 16) ^ (row % 16), so a wave instruction fills 4 whole rows and the
//    fragment reads (16 rows at one k-chunk) fall in 16 different 16-byte bank groups;
//  * lane (j = l % 16, g = l / 16) holds column j of its tiles and loads quant block g of the step
//    and its scale into a ring of 4 register stages; MFMA k-slice s takes word s of that block, so
//    the A fragment of lane (j, g) in slice s is row j at k-chunk 4g + s;
//  * loads of a step past the workgroup's range carry out-of-range buffer offsets (no memory
//    access), so every step issues the same loads and the explicit vector-memory waits are exact;
//  * SILU (gate_up with rows interleaved in groups of 16, see k_gemm_w4m): mid = f16(silu(g) u), g
//    and u rounded to f16 first.  With NT even a wave's tiles 2u and 2u + 1 hold gate and up of the
//    same 16 outputs; with NT = 1 the pairs are in neighbouring waves and meet in LDS.
template <int MT, int NT, bool PARTIAL, bool SILU = false>
__global__ __launch_bounds__(256) void k_gemm_w4p(const f16* __restrict__ A, const uint32_t* __restrict__ W,
                                                  const f16* __restrict__ S, f16* __restrict__ Y,
                                                  float* __restrict__ part, int M, int N, int K, int ks_tiled) {
    constexpr int BM = MT * 16;
    constexpr int BN = 4 * NT * 16;
    const int ksplit = ks_tiled >> 1, tiled = ks_tiled & 1;
    constexpr int STAGE = BM * 256;           // bytes of one A stage (128 k of BM rows)
    constexpr int NLD = MT;                   // direct-to-LDS loads per thread per step
    constexpr int PER_STEP = NLD + 2 * NT;    // vector-memory loads a thread issues per step
    constexpr int WAIT2 = vmcnt_imm(2 * PER_STEP);
    __shared__ __attribute__((aligned(1024))) uint8_t As0[STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t As1[STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t As2[STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t As3[STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, g = lane >> 4;
    int bx, by, bz;
    // the launch grid (ceil(N / BN), ceil(M / BM), ksplit) from the arguments, not from the dispatch
    // packet's grid size (one more scalar load before the first weight load could be issued)
    xcd_tile(blockIdx.x + (N + BN - 1) / BN * (blockIdx.y + (M + BM - 1) / BM * blockIdx.z), (N + BN - 1) / BN,
             (M + BM - 1) / BM, ksplit, bx, by, bz);
    const int m0 = by * BM, n0 = bx * BN;
    const int KB = K >> 5;
    const int steps = K / KSTEP / ksplit;  // a multiple of 4 (checked by the launcher)
    const int step0 = bz * steps;

    const Rsrc ra = make_rsrc(A, (uint32_t)M * K * 2), rw = make_rsrc(W, (uint32_t)N * K / 2),
               rs = make_rsrc(S, (uint32_t)N * KB * 2);
    uint32_t aoff[NLD];
#pragma unroll
    for (int i = 0; i < NLD; i++) {
        const int q = (i * 4 + wave) * 64 + lane;
        const int row = q >> 4, c = (q & 15) ^ (row & 15);
        aoff[i] = (uint32_t)(min(m0 + row, M - 1) * K + c * 8) * 2u;
    }
    // fragment read of tile a, slice s: row 16a + j, k-chunk 4g + s
    uint32_t foff[MT][4];
#pragma unroll
    for (int a = 0; a < MT; a++)
#pragma unroll
        for (int s = 0; s < 4; s++) foff[a][s] = (a * 16 + j) * 256 + (((4 * g + s) ^ j) << 4);

    int ncol[NT];
    uint32_t woff[NT], soff[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        ncol[t] = n0 + (wave * NT + t) * 16 + j;
        const uint32_t n = (uint32_t)min(ncol[t], N - 1);
        const uint32_t i0 = tiled ? ((n >> 5) * (uint32_t)(KB >> 1) + (g >> 1)) * 64 + (n & 31) * 2 + (g & 1) : n * KB + g;
        woff[t] = i0 * 16u;
        soff[t] = i0 * 2u;
    }
    const uint32_t wstep = tiled ? 2048u : 64u, sstep = tiled ? 256u : 8u;

    f32x4 acc[MT][NT];
#pragma unroll
    for (int a = 0; a < MT; a++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[a][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 bw[4][NT];
    uint32_t bs[4][NT];
    auto issue = [&](int it, uint8_t* dst, u32x4* bwd, uint32_t* bsd) {
        const bool in = it < steps;
        const uint32_t ka = in ? (uint32_t)(step0 + it) * KSTEP * 2 : OOB;
        const uint32_t kw = in ? (uint32_t)(step0 + it) * wstep : OOB;
        const uint32_t ks_ = in ? (uint32_t)(step0 + it) * sstep : OOB;
#pragma unroll
        for (int i = 0; i < NLD; i++) buf_lds16(ra, aoff[i], ka, dst + (i * 4 + wave) * 1024);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            bwd[t] = buf_b128(rw, woff[t], kw);
            bsd[t] = buf_b16(rs, soff[t], ks_);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    auto frag = [&](const uint8_t* cur, int s, f16x8* af) {
#pragma unroll
        for (int a = 0; a < MT; a++) af[a] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(cur + foff[a][s]));
    };
    auto deq = [&](const u32x4* bwc, const uint32_t* bsc, int s, f16x8* bf) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const f16 scv = __builtin_bit_cast(f16, (uint16_t)bsc[t]);
            const f16x2 sc2 = f16x2{scv, scv};
            f16x2 p0, p1, p2, p3;
            nib_pairs(bwc[t][s], p0, p1, p2, p3);
            bf[t] = cat4(p0 * sc2, p1 * sc2, p2 * sc2, p3 * sc2);
        }
    };
    // Step it reads stage `cur` and refills stage `fill` (read at it - 1) for step it + 3; slice
    // s + 1's fragments and weights are produced while slice s's MFMAs run.
    auto step = [&](const uint8_t* cur, uint8_t* fill, const u32x4* bwc, const uint32_t* bsc, u32x4* bwf,
                    uint32_t* bsf, int it) {
        issue(it + 3, fill, bwf, bsf);
        f16x8 af[2][MT], bf[2][NT];
        frag(cur, 0, af[0]);
        deq(bwc, bsc, 0, bf[0]);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int cu = s & 1, nx = cu ^ 1;
            if (s < 3) {
                frag(cur, s + 1, af[nx]);
                deq(bwc, bsc, s + 1, bf[nx]);
            }
#pragma unroll
            for (int a = 0; a < MT; a++)
#pragma unroll
                for (int t = 0; t < NT; t++)
                    acc[a][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[cu][a], bf[cu][t], acc[a][t], 0, 0, 0);
        }
        wait_loads<WAIT2>();  // the loads of steps it + 2, it + 3 may still be in flight
        bar_noflush();
    };

    issue(0, As0, bw[0], bs[0]);
    issue(1, As1, bw[1], bs[1]);
    issue(2, As2, bw[2], bs[2]);
    wait_loads<WAIT2>();
    bar_noflush();
    int it = 0;
    do {
        step(As0, As3, bw[0], bs[0], bw[3], bs[3], it);
        step(As1, As0, bw[1], bs[1], bw[0], bs[0], it + 1);
        step(As2, As1, bw[2], bs[2], bw[1], bs[1], it + 2);
        step(As3, As2, bw[3], bs[3], bw[2], bs[2], it + 3);
        it += 4;
    } while (it < steps);
    wait_loads<vmcnt_imm(0)>();  // the trailing out-of-range loads, before the workgroup ends

    // Output: acc[a][t][r] is row m0 + 16a + 4g + r, column ncol[t].
    if constexpr (SILU) {
        const int ow = N >> 1;
        if constexpr (NT % 2 == 0) {
#pragma unroll
            for (int u = 0; u < NT / 2; u++) {
                const int cb = n0 + (wave * NT + 2 * u) * 16;
                if (cb >= N) continue;
#pragma unroll
                for (int a = 0; a < MT; a++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int m = m0 + a * 16 + g * 4 + r;
                        const float gv = (float)(f16)acc[a][2 * u][r], uv = (float)(f16)acc[a][2 * u + 1][r];
                        if (m < M) Y[(size_t)m * ow + (cb >> 1) + j] = (f16)silu_mul(gv, uv);
                    }
            }
        } else {
            static_assert(NT == 1, "odd tile counts: one tile per wave");
            // staged as f16 rows of 64 gate/up columns (+ 8 halves of padding); wave w's tile is
            // columns 16w .. 16w + 15, so waves 2v and 2v + 1 hold gate and up of mid columns 16v ..
            constexpr int LDW = 72;
            static_assert(BM * LDW * 2 <= STAGE, "the staged tile fits one ring stage");
            f16* st = reinterpret_cast<f16*>(As0);
            lds_barrier();  // every wave's ring reads and loads are done
#pragma unroll
            for (int a = 0; a < MT; a++)
#pragma unroll
                for (int r = 0; r < 4; r++) st[(a * 16 + g * 4 + r) * LDW + wave * 16 + j] = (f16)acc[a][0][r];
            lds_barrier();
#pragma unroll
            for (int e = 0; e < BM / 8; e++) {
                const int idx = e * 256 + tid, row = idx >> 5, mc = idx & 31, v = mc >> 4, jj = mc & 15;
                const int m = m0 + row;
                const float gv = (float)st[row * LDW + 32 * v + jj], uv = (float)st[row * LDW + 32 * v + 16 + jj];
                if (m < M && n0 + 32 * v < N) Y[(size_t)m * ow + (n0 >> 1) + mc] = (f16)silu_mul(gv, uv);
            }
        }
        return;
    }
    if constexpr (!PARTIAL) {
#pragma unroll
        for (int a = 0; a < MT; a++)
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = m0 + a * 16 + g * 4 + r;
                    if (m < M && ncol[t] < N) Y[(size_t)m * N + ncol[t]] = (f16)acc[a][t][r];
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
                if (m < M && ncol[t] < N) __builtin_nontemporal_store(acc[a][t][r], mine + (size_t)m * N + ncol[t]);
            }
}

// The same product on v_mfma_f32_32x32x16_f16 (measured on MI355X: 2.2 PFLOP/s with 4 independent
// accumulators per wave; the 16x16x32 form needs 16 to get close).  Prefill and batched questions
// (f16 dequant).
//  * a wave owns MT2 32-row tiles x NT2 32-column tiles; 4 waves side by side along N, so every
//    dequantized weight feeds MT2 MFMAs (at MT2 = 4: 3 VALU per MFMA, which the MFMA pipe hides);
//  * k advances in steps of 64 through a ring of 4 LDS stages, loads issued 3 steps ahead (the
//    first touch of a weight block or an A row comes from HBM, a few microseconds under load);
//    one barrier per step;
//  * the A tile of a step (BM rows x 128 B) is fetched straight into LDS (buffer_load_dwordx4 lds):
//    16-byte chunk q of the stage (q = (i * 4 + wave) * 64 + lane for the thread's i-th load) holds
//    row q / 8, k-chunk (q % 8) ^ ((row / 2) % 8).  A wave instruction fills 1 KiB (8 whole rows),
//    and the fragment reads (16 rows at one k-chunk per 16 lanes) cover all 64 banks;
//  * lane (r = l % 32, g = l / 32) holds column r of its column tiles and loads quant block g of the
//    step (16 bytes) and its scale, up to 3 steps ahead in registers; MFMA k-slice s (16 k) takes
//    word s of that block, which is k-chunk 4g + s of the step, so the A fragment of lane (r, g) is
//    the 8 halves of row r at that k-chunk (the engine nibble order makes them natural);
//  * D of the 32x32 tile: register i of lane l is D row 8(i/4) + 4(l/32) + i%4, D column l%32.
//    Split-K partials (PARTIAL) take A as the row operand: lane l holds output column l%32 of 16
//    rows, stored as single floats (a store instruction covers 32 columns of 2 rows).  f16 outputs
//    take the weights as the row operand (the same fragments, swapped): lane (r, g) holds output
//    row r and the columns 8j + 4g .. 8j + 4g + 3 of its tile in registers 4j .. 4j + 3;
//  * the end of a kernel writes the dirty L2 lines back (the next kernel may run on another XCD),
//    and every workgroup finishes at about the same time, so the output is written in one burst
//    after the last MFMA.  f16 outputs go through the (then free) LDS ring as f32 and leave as
//    whole-row 16-byte non-temporal stores; partials are stored non-temporally;
//  * KH = 2 (NT2 = 1): 8 waves, two halves of 4 that take the first and the second half of the
//    workgroup's k steps, each with its own ring; at the end the second half hands its
//    accumulators to the first through LDS.  The k chain per wave halves and every SIMD holds two
//    waves, for grids of about one workgroup per CU (batched questions, split-K prefill shapes);
//  * SILU (gate_up, unsplit): W holds gate_up with its rows interleaved in groups of 16 (rows
//    32p .. 32p + 15 are gate rows 16p .., the next 16 the matching up rows, interleave_gate_up),
//    so registers k and 8 + k of a lane hold gate and up of one output element (row r, mid column
//    16p + 8(k/4) + 4g + k%4); Y = mid[M][N / 2] = f16(silu(g) * u), g and u rounded to f16 first
//    as the reference stores them.
template <int MT2, int NT2, bool PARTIAL, bool SILU = false, int KH = 1>
__global__ __attribute__((amdgpu_flat_work_group_size(256 * KH, 256 * KH), amdgpu_waves_per_eu(2))) void k_gemm_w4m(
    const f16* __restrict__ A, const uint32_t* __restrict__ W, const f16* __restrict__ S, f16* __restrict__ Y,
    float* __restrict__ part, int M, int N, int K, int ks_tiled) {
    constexpr int KS = 64;                   // k per step
    constexpr int BM = MT2 * 32;
    constexpr int BN = 4 * NT2 * 32;
    const int ksplit = ks_tiled >> 1, tiled = ks_tiled & 1;
    constexpr int STAGE = BM * KS * 2;       // bytes of one A stage
    constexpr int NLD = BM / 32;             // direct-to-LDS loads per thread per step
    constexpr int PER_STEP = NLD + 2 * NT2;  // vector-memory loads a thread issues per step
    constexpr int WAIT2 = 0x0F70 | ((2 * PER_STEP) & 15) | (((2 * PER_STEP) >> 4) << 14);  // vmcnt(2 steps)
    // One array per stage, so the compiler can see that the loads into one stage never alias the
    // fragment reads of another.
    static_assert(KH == 1 || KH == 2, "one or two k halves");
    __shared__ __attribute__((aligned(1024))) uint8_t As0[KH * STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t As1[KH * STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t As2[KH * STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t As3[KH * STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wall = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kh = wall >> 2, wave = wall & 3;  // k half, wave within the half
    const int r = lane & 31, g = lane >> 5;
    // this half's ring: stage i at Asi + kh * STAGE
    uint8_t* const R0 = As0 + kh * STAGE;
    uint8_t* const R1 = As1 + kh * STAGE;
    uint8_t* const R2 = As2 + kh * STAGE;
    uint8_t* const R3 = As3 + kh * STAGE;
    int bx, by, bz;
    // the launch grid (ceil(N / BN), ceil(M / BM), ksplit) from the arguments, not from the dispatch
    // packet's grid size (one more scalar load before the first weight load could be issued)
    xcd_tile(blockIdx.x + (N + BN - 1) / BN * (blockIdx.y + (M + BM - 1) / BM * blockIdx.z), (N + BN - 1) / BN,
             (M + BM - 1) / BM, ksplit, bx, by, bz);
    const int m0 = by * BM, n0 = bx * BN;
    const int KB = K >> 5;
    const int steps = (K / KS) / ksplit / KH;  // a multiple of 4 (checked by the launcher)
    const int step0 = (bz * KH + kh) * steps;

    // Loads go through buffer resources: per-lane offsets fixed for the whole k loop, the step in the
    // uniform offset.  A step past this workgroup's range gets an offset past the buffer (no memory
    // access), so every step issues the same loads and the wait counts below are exact.
    const Rsrc ra = make_rsrc(A, (uint32_t)M * K * 2), rw = make_rsrc(W, (uint32_t)N * K / 2),
               rs = make_rsrc(S, (uint32_t)N * KB * 2);
    // A: this thread's chunks of a step (rows past M read the last row; their outputs are never
    // stored).
    uint32_t aoff[NLD];
#pragma unroll
    for (int i = 0; i < NLD; i++) {
        const int q = (i * 4 + wave) * 64 + lane;
        const int row = q >> 3, c = (q & 7) ^ ((row >> 1) & 7);
        aoff[i] = (uint32_t)(min(m0 + row, M - 1) * K + c * 8) * 2u;
    }
    // Fragment reads: LDS byte offset of row r, k-chunk 4g + s (tile a adds a * 4 KiB).
    uint32_t foff[4];
#pragma unroll
    for (int s = 0; s < 4; s++) foff[s] = r * 128 + (((4 * g + s) ^ ((r >> 1) & 7)) << 4);

    // Block g of step 0 of column n (plain: n * KB + g; tiled: inside column tile n / 32), and the
    // bytes one step advances the weight and scale offsets.
    int ncol[NT2];
    uint32_t woff[NT2], soff[NT2];
#pragma unroll
    for (int t = 0; t < NT2; t++) {
        ncol[t] = n0 + (wave * NT2 + t) * 32 + r;
        const uint32_t n = (uint32_t)min(ncol[t], N - 1);
        const uint32_t i0 = tiled ? (n >> 5) * (uint32_t)(KB >> 1) * 64 + (n & 31) * 2 + g : n * KB + g;
        woff[t] = i0 * 16u;
        soff[t] = i0 * 2u;
    }
    const uint32_t wstep = tiled ? 1024u : 32u, sstep = tiled ? 128u : 4u;

    f32x16 acc[MT2][NT2];
#pragma unroll
    for (int a = 0; a < MT2; a++)
#pragma unroll
        for (int t = 0; t < NT2; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[a][t][i] = 0.f;

    // Weight blocks and scales of the 4 steps in flight (ring index = step % 4).  A scale is kept in
    // a register of its own: packing two per register would wait for the load at once.
    u32x4 bw[4][NT2];
    uint32_t bs[4][NT2];
    auto issue = [&](int it, uint8_t* dst, u32x4* bwd, uint32_t* bsd) {
        const bool in = it < steps;
        const uint32_t ka = in ? (uint32_t)(step0 + it) * KS * 2 : 0x80000000u;
        const uint32_t kw = in ? (uint32_t)(step0 + it) * wstep : 0x80000000u;
        const uint32_t ks_ = in ? (uint32_t)(step0 + it) * sstep : 0x80000000u;
#pragma unroll
        for (int i = 0; i < NLD; i++) buf_lds16(ra, aoff[i], ka, dst + (i * 4 + wave) * 1024);
#pragma unroll
        for (int t = 0; t < NT2; t++) {
            bwd[t] = buf_b128(rw, woff[t], kw);
            bsd[t] = buf_b16(rs, soff[t], ks_);
        }
        // each step's loads stay together and in step order, also in the prologue
        __builtin_amdgcn_sched_barrier(0);
    };
    auto frag = [&](const uint8_t* cur, int s, f16x8* af) {
#pragma unroll
        for (int a = 0; a < MT2; a++)
            af[a] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(cur + a * 4096 + foff[s]));
    };
    auto deq = [&](const u32x4* bwc, const uint32_t* bsc, int s, f16x8* bf) {
#pragma unroll
        for (int t = 0; t < NT2; t++) {
            const f16 scv = __builtin_bit_cast(f16, (uint16_t)bsc[t]);
            const f16x2 sc2 = f16x2{scv, scv};
            f16x2 p0, p1, p2, p3;
            nib_pairs(bwc[t][s], p0, p1, p2, p3);
            bf[t] = cat4(p0 * sc2, p1 * sc2, p2 * sc2, p3 * sc2);
        }
    };
    // Step it reads stage `cur` and refills stage `fill` (the one read at it - 1) for step it + 3.
    // Software pipeline: the A fragments and dequantized weights of k-slice s + 1 are produced while
    // the MFMAs of slice s run (the last slice dequantizes the next step's first one into bf0), with
    // the issue order pinned: per MFMA a share of the dequant VALU work and one fragment read.
    // Before the barrier every thread waits for its loads of step it + 1.
    constexpr int NMF = MT2 * NT2;                  // MFMAs per k-slice
    constexpr int VPER = (13 * NT2 + NMF - 1) / NMF;  // dequant VALU instructions per MFMA
    auto step = [&](const uint8_t* cur, uint8_t* fill, const u32x4* bwc, const uint32_t* bsc, const u32x4* bwn,
                    const uint32_t* bsn, u32x4* bwf, uint32_t* bsf, f16x8* bf0, int it) {
        issue(it + 3, fill, bwf, bsf);
        f16x8 af[2][MT2], bf[2][NT2];
#pragma unroll
        for (int t = 0; t < NT2; t++) bf[0][t] = bf0[t];
        frag(cur, 0, af[0]);
        __builtin_amdgcn_sched_group_barrier(0x100, MT2, 0);  // the first slice's fragment reads
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int cu = s & 1, nx = cu ^ 1;
            if (s < 3) {
                frag(cur, s + 1, af[nx]);
                deq(bwc, bsc, s + 1, bf[nx]);
            } else {
                deq(bwn, bsn, 0, bf0);
            }
#pragma unroll
            for (int a = 0; a < MT2; a++)
#pragma unroll
                for (int t = 0; t < NT2; t++)
                    acc[a][t] = PARTIAL ? __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cu][a], bf[cu][t], acc[a][t], 0, 0, 0)
                                        : __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[cu][t], af[cu][a], acc[a][t], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < NMF; j++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);     // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, VPER, 0);  // VALU
                if (s < 3 && j < MT2) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // a fragment read
            }
        }
        wait_loads<WAIT2>();  // the loads of steps it + 2, it + 3 may still be in flight
        bar_noflush();
    };

    issue(0, R0, bw[0], bs[0]);
    issue(1, R1, bw[1], bs[1]);
    issue(2, R2, bw[2], bs[2]);
    wait_loads<WAIT2>();
    bar_noflush();
    f16x8 bf0[NT2];
    deq(bw[0], bs[0], 0, bf0);
    // steps >= 4: no zero-trip branch, which would let the compiler sink the prologue's weight loads
    // past the first wait (and so change what it counts).
    int it = 0;
    do {
        step(R0, R3, bw[0], bs[0], bw[1], bs[1], bw[3], bs[3], bf0, it);
        step(R1, R0, bw[1], bs[1], bw[2], bs[2], bw[0], bs[0], bf0, it + 1);
        step(R2, R1, bw[2], bs[2], bw[3], bs[3], bw[1], bs[1], bf0, it + 2);
        step(R3, R2, bw[3], bs[3], bw[0], bs[0], bw[2], bs[2], bf0, it + 3);
        it += 4;
    } while (it < steps);
    wait_loads<0x0F70>();  // the trailing out-of-range loads, before the LDS is released

    if constexpr (KH == 2) {
        // The second half's accumulators go to the first half's wave of the same columns through the
        // second half of that wave's ring array (lane-major 16-byte chunks, conflict-free), one column
        // tile per pass (a pass is MT2 x 4 KiB, at most the STAGE bytes there).
        uint8_t* const xr = (wave == 0 ? As0 : wave == 1 ? As1 : wave == 2 ? As2 : As3) + STAGE;
#pragma unroll
        for (int t = 0; t < NT2; t++) {
            lds_barrier();  // every wave's loads have landed (the rings are free), or the last pass is read
            if (kh == 1) {
#pragma unroll
                for (int a = 0; a < MT2; a++)
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        *reinterpret_cast<f32x4*>(xr + ((a * 4 + q) * 64 + lane) * 16) =
                            f32x4{acc[a][t][4 * q], acc[a][t][4 * q + 1], acc[a][t][4 * q + 2], acc[a][t][4 * q + 3]};
            }
            lds_barrier();
            if (kh == 0) {
#pragma unroll
                for (int a = 0; a < MT2; a++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const f32x4 v = *reinterpret_cast<const f32x4*>(xr + ((a * 4 + q) * 64 + lane) * 16);
#pragma unroll
                        for (int e = 0; e < 4; e++) acc[a][t][4 * q + e] += v[e];
                    }
            }
        }
    }
    // From here on the first half (threads 0 .. 255) stores; the second half only joins the
    // barriers of the staged path.
    const bool act = kh == 0;

    if constexpr (PARTIAL) {
        if (!act) return;
        float* mine = part + (size_t)bz * M * N;
#pragma unroll
        for (int a = 0; a < MT2; a++)
#pragma unroll
            for (int t = 0; t < NT2; t++) {
                if (ncol[t] >= N) continue;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int m = m0 + a * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
                    if (m < M) __builtin_nontemporal_store(acc[a][t][i], mine + (size_t)m * N + ncol[t]);
                }
            }
        return;
    }
    // f16 outputs: row m0 + 32a + r, columns cb + 8j + 4g + e of column tile cb.  With every output
    // row 16-byte aligned they leave as 16-byte stores: staged through LDS for prefill-sized M, else
    // straight from registers after v_permlane32_swap has given lane (r, 0) the 8 columns 16h .. 16h
    // + 7 and lane (r, 1) the next 8 (h = 0, 1; the swap exchanges the upper 32 lanes of its first
    // operand with the lower 32 lanes of its second).  Otherwise element by element.
    const int ow = SILU ? N >> 1 : N;  // output row width
    const bool vec = ow % 8 == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0;
    const bool staged = vec && M >= 256;  // measured: direct stores win for a lone workgroup per CU
    if (!staged) {
        if (!act) return;
#pragma unroll
        for (int a = 0; a < MT2; a++)
#pragma unroll
            for (int t = 0; t < NT2; t++) {
                const int cb = n0 + (wave * NT2 + t) * 32, m = m0 + a * 32 + r;
                if (cb >= N) continue;  // wave-uniform
                if (vec) {
                    // P[2j + e/2] packs columns 8j + 4g + e, e + 1 (SILU: the 8 outputs, 2 per register)
                    uint32_t P[8];
                    if constexpr (SILU) {
#pragma unroll
                        for (int k = 0; k < 8; k += 2) {
                            f16 o[2];
#pragma unroll
                            for (int u = 0; u < 2; u++) {
                                const float gv = (float)(f16)acc[a][t][k + u], uv = (float)(f16)acc[a][t][8 + k + u];
                                o[u] = (f16)silu_mul(gv, uv);
                            }
                            P[k / 2] = __builtin_bit_cast(uint32_t, f16x2{o[0], o[1]});
                        }
                    } else {
#pragma unroll
                        for (int k = 0; k < 16; k += 2)
                            P[k / 2] = __builtin_bit_cast(uint32_t, f16x2{(f16)acc[a][t][k], (f16)acc[a][t][k + 1]});
                    }
                    constexpr int NH = SILU ? 1 : 2;  // 16-column halves of the tile's outputs
#pragma unroll
                    for (int h = 0; h < NH; h++) {
#pragma unroll
                        for (int e = 0; e < 2; e++) {
                            const auto sw = __builtin_amdgcn_permlane32_swap(P[4 * h + e], P[4 * h + 2 + e], false, false);
                            P[4 * h + e] = sw[0];
                            P[4 * h + 2 + e] = sw[1];
                        }
                        const int n = (SILU ? cb >> 1 : cb) + 16 * h + 8 * g;
                        if (m < M && n < ow)
                            __builtin_nontemporal_store(u32x4{P[4 * h], P[4 * h + 1], P[4 * h + 2], P[4 * h + 3]},
                                                        reinterpret_cast<u32x4*>(Y + (size_t)m * ow + n));
                    }
                    continue;
                }
                if (m >= M) continue;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    if constexpr (SILU) {
                        if (i >= 8) continue;  // N % 32 == 0: the tile is whole
                        const float gv = (float)(f16)acc[a][t][i], uv = (float)(f16)acc[a][t][8 + i];
                        const int j = (cb >> 1) + 8 * (i >> 2) + 4 * g + (i & 3);
                        Y[(size_t)m * ow + j] = (f16)silu_mul(gv, uv);
                    } else {
                        const int n = cb + 8 * (i >> 2) + 4 * g + (i & 3);
                        if (n < N) Y[(size_t)m * N + n] = (f16)acc[a][t][i];
                    }
                }
            }
        return;
    }
    // One pass per column tile t of the waves.  Wave w writes its 32 columns of the pass into stage
    // w: f32 rows of 128 B, 16-byte chunk q of row rho at (q ^ (rho / 2) % 8) (conflict-free
    // ds_write_b128 over 16 lanes); SILU writes its 16 f16 outputs, rows of 32 B.  Then each thread
    // reads 8 consecutive outputs of one row and stores them with one 16-byte store.
    uint8_t* const wst = wave == 0 ? As0 : wave == 1 ? As1 : wave == 2 ? As2 : As3;
#pragma unroll
    for (int t = 0; t < NT2; t++) {
        lds_barrier();  // the ring (or the previous pass) is free: every wave's loads have landed
#pragma unroll
        for (int a = 0; a < MT2; a++) {
            if (!act) break;
            const int rho = 32 * a + r;
            if constexpr (SILU) {
                f16 o[8];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const float gv = (float)(f16)acc[a][t][k], uv = (float)(f16)acc[a][t][8 + k];
                    o[k] = (f16)silu_mul(gv, uv);
                }
                *reinterpret_cast<f16x4*>(wst + rho * 32 + 8 * g) = f16x4{o[0], o[1], o[2], o[3]};
                *reinterpret_cast<f16x4*>(wst + rho * 32 + 16 + 8 * g) = f16x4{o[4], o[5], o[6], o[7]};
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int q = (2 * j + g) ^ ((rho >> 1) & 7);
                    *reinterpret_cast<f32x4*>(wst + rho * 128 + q * 16) =
                        f32x4{acc[a][t][4 * j], acc[a][t][4 * j + 1], acc[a][t][4 * j + 2], acc[a][t][4 * j + 3]};
                }
            }
        }
        lds_barrier();
        if (!act) continue;
        if constexpr (SILU) {
            // a mid row of the pass: 4 waves x 16 outputs = 8 chunks
            const int c = tid & 7, w = c >> 1;
            const uint8_t* src = w == 0 ? As0 : w == 1 ? As1 : w == 2 ? As2 : As3;
            const int cb = n0 + (w * NT2 + t) * 32, j = (cb >> 1) + 8 * (c & 1);
#pragma unroll
            for (int it = 0; it < MT2; it++) {
                const int rho = it * 32 + (tid >> 3), m = m0 + rho;
                const f16x8 v = *reinterpret_cast<const f16x8*>(src + rho * 32 + 16 * (c & 1));
                if (m < M && cb < N) __builtin_nontemporal_store(v, reinterpret_cast<f16x8*>(Y + (size_t)m * ow + j));
            }
        } else {
            // an output row of the pass: 4 waves x 32 columns = 16 groups of 8
            const int cp = tid & 15, w = cp >> 2, q = 2 * (cp & 3);
            const uint8_t* src = w == 0 ? As0 : w == 1 ? As1 : w == 2 ? As2 : As3;
            const int n = n0 + (w * NT2 + t) * 32 + 8 * (cp & 3);
#pragma unroll
            for (int it = 0; it < MT2 * 2; it++) {
                const int rho = it * 16 + (tid >> 4), m = m0 + rho, sw = (rho >> 1) & 7;
                const f32x4 v0 = *reinterpret_cast<const f32x4*>(src + rho * 128 + ((q ^ sw) * 16));
                const f32x4 v1 = *reinterpret_cast<const f32x4*>(src + rho * 128 + (((q + 1) ^ sw) * 16));
                const f16x8 h = f16x8{(f16)v0[0], (f16)v0[1], (f16)v0[2], (f16)v0[3],
                                      (f16)v1[0], (f16)v1[1], (f16)v1[2], (f16)v1[3]};
                if (m < M && n < N) __builtin_nontemporal_store(h, reinterpret_cast<f16x8*>(Y + (size_t)m * N + n));
            }
        }
    }
}

// In-place rewrite of int4 weight words from the reference's nibble order (k = 8w + e of a quant
// block at bits 4e of word w) to the engine's: nibble position p holds e = [0,2,4,6,1,3,5,7][p],
// so that nib_pairs yields the pairs (k0,k1), (k2,k3), (k4,k5), (k6,k7) in natural k order.
__global__ void k_repack_w4(uint32_t* __restrict__ W, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t o = W[i];
    uint32_t w = 0;
#pragma unroll
    for (int p = 0; p < 8; p++) {
        const int e = p < 4 ? 2 * p : 2 * (p - 4) + 1;
        w |= ((o >> (4 * e)) & 15u) << (4 * p);
    }
    W[i] = w;
}

// dst row n of a [N][K] int4 matrix (16-byte blocks and f16 scales) = src row gate_up_row(n): groups
// of 32 rows alternate 16 gate rows and the 16 matching up rows (N = 2I).
__device__ __forceinline__ int gate_up_row(int n, int N) {
    const int p = n >> 5, w = n & 31;
    return w < 16 ? 16 * p + w : (N >> 1) + 16 * p + (w - 16);
}
// dst = src in the tiled layout (one thread per 16-byte block and its scale)
__global__ void k_tile_w4(const u32x4* __restrict__ sw, const f16* __restrict__ ss, u32x4* __restrict__ dw,
                          f16* __restrict__ ds, int N, int KB) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)N * KB) return;
    const size_t n = i / KB, b = i % KB;
    const size_t o = ((n >> 5) * (size_t)(KB >> 1) + (b >> 1)) * 64 + (n & 31) * 2 + (b & 1);
    dw[o] = sw[i];
    ds[o] = ss[i];
}

__global__ void k_interleave_gate_up(const u32x4* __restrict__ sw, const f16* __restrict__ ss, u32x4* __restrict__ dw,
                                     f16* __restrict__ ds, int N, int KB) {
    const int n = blockIdx.x, src = gate_up_row(n, N);
    for (int b = threadIdx.x; b < KB; b += blockDim.x) {
        dw[(size_t)n * KB + b] = sw[(size_t)src * KB + b];
        ds[(size_t)n * KB + b] = ss[(size_t)src * KB + b];
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

// Kernel arguments: A, W, S, Y, part, M, N, K, split count << 1 | tiled layout (14 dwords, all of
// them preloaded into SGPRs before the waves start).
typedef void (*GemmFn)(const f16*, const uint32_t*, const f16*, f16*, float*, int, int, int, int);
struct Cfg {
    int mt, nt;
    bool exact;
    GemmFn f16_out, part_out;
    bool wide;  // k_gemm_w4m (k steps of 64 in a ring of 4)
    GemmFn silu_out;  // the SiLU * mul epilogue (k_gemm_w4m and k_gemm_w4p configurations)
    int kh;           // k halves per workgroup (256 threads each)
    bool pipe = false;  // k_gemm_w4p (loads three 128-k steps ahead; k steps per split a multiple of 4)
};

#define SD_CFG(MT, NT, EX) Cfg{MT, NT, EX, k_gemm_w4<MT, NT, EX, false>, k_gemm_w4<MT, NT, EX, true>, false, nullptr, 1}
#define SD_CFGM(MT2, NT2)                                                                                        \
    Cfg{2 * MT2, 2 * NT2, false, k_gemm_w4m<MT2, NT2, false>, k_gemm_w4m<MT2, NT2, true>, true,                  \
        k_gemm_w4m<MT2, NT2, false, true>, 1}
#define SD_CFGMH(MT2)                                                                                            \
    Cfg{2 * MT2, 2, false, k_gemm_w4m<MT2, 1, false, false, 2>, k_gemm_w4m<MT2, 1, true, false, 2>, true,        \
        k_gemm_w4m<MT2, 1, false, true, 2>, 2}
#define SD_CFGP(MT, NT)                                                                                    \
    Cfg{MT, NT, false, k_gemm_w4p<MT, NT, false>, k_gemm_w4p<MT, NT, true>, false,                          \
        k_gemm_w4p<MT, NT, false, true>, 1, true}
#define SD_CFGMH2(MT2)                                                                                           \
    Cfg{2 * MT2, 4, false, k_gemm_w4m<MT2, 2, false, false, 2>, k_gemm_w4m<MT2, 2, true, false, 2>, true,        \
        k_gemm_w4m<MT2, 2, false, true, 2>, 2}
const Cfg kCfgs[] = {
    SD_CFG(1, 1, true), SD_CFG(2, 1, true),                                           // M <= 20: f32 dequant
    SD_CFG(1, 1, false), SD_CFG(2, 1, false), SD_CFG(3, 1, false), SD_CFG(4, 1, false),  // skinny
    SD_CFG(8, 2, false), SD_CFG(8, 4, false), SD_CFG(4, 2, false), SD_CFG(8, 1, false),  // prefill
    SD_CFG(4, 4, false), SD_CFG(6, 2, false), SD_CFG(3, 2, false), SD_CFG(2, 2, false),
    SD_CFG(4, 3, false), SD_CFG(3, 3, false), SD_CFG(2, 3, false), SD_CFG(5, 2, false),
    // 32x32x16 MFMA tiles (MT2 x 32 rows, 4 x NT2 x 32 columns), listed in 16-row / 64-column units
    SD_CFGM(2, 1), SD_CFGM(2, 2), SD_CFGM(4, 1), SD_CFGM(3, 1), SD_CFGM(1, 1), SD_CFGM(4, 2),
    // the same with two k halves per workgroup (512 threads): (2,1), (4,1), (3,1)
    SD_CFGMH(2), SD_CFGMH(4), SD_CFGMH(3),
    // two column tiles per wave with two k halves: (4,2), (2,2)
    SD_CFGMH2(4), SD_CFGMH2(2),
    // 16x16 tiles with loads three steps ahead: (1,1), (2,1), (3,1), (4,1), (2,2), (3,2), (4,2), (1,2)
    SD_CFGP(1, 1), SD_CFGP(2, 1), SD_CFGP(3, 1), SD_CFGP(4, 1), SD_CFGP(2, 2), SD_CFGP(3, 2), SD_CFGP(4, 2),
    SD_CFGP(1, 2),
};
#undef SD_CFG
#undef SD_CFGM
#undef SD_CFGMH
#undef SD_CFGMH2
#undef SD_CFGP
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

int pick_cfg(int M, bool exact) {
    if (exact) return M <= 16 ? 0 : 1;
    if (M <= 16) return 2;
    if (M <= 32) return 3;
    if (M <= 48) return 4;
    if (M <= 64) return 5;
    return 8;  // (4, 2): the best prefill tile on MI355X in a sweep over the 2B's shapes
}

// Configuration indices into kCfgs used by the planner: the 64-wide-step 32x32 MFMA tiles (need K a
// multiple of 256), the same with two k halves per workgroup (K a multiple of 512), and 16x16 tiles.
constexpr int W21 = 18, W22 = 19, W41 = 20, W31 = 21, W42 = 23, W21h = 24, W41h = 25, W31h = 26;
constexpr int T21 = 3, T31 = 4, T41 = 5;  // 16x16 (2,1), (3,1), (4,1)
// 16x16, loads three steps ahead: (2,1), (3,1), (4,1), (2,2), (3,2)
constexpr int P21 = 30, P31 = 31, P41 = 32, P22 = 33, P32 = 34;

// Measured plans for the 2B hybrid's five matmul shapes at M = 256 .. 2560 (entry i for M in
// (192 + 64 i, 256 + 64 i]): each configuration and split timed on MI355X with the weights cold (24
// copies rotated, more than the 256 MB last-level cache holds, as a forward streams its layers'),
// two runs on two boxes averaged; a split plan is charged the consumer's read of its f32 slots (at
// 5 TB/s); an entry differs from the rules below only where it was at least 3 % faster.  The grid's
// fill of the 256 CUs decides most entries: the best tile moves with M as the workgroup count
// crosses multiples of one or two workgroups per CU.
constexpr int kPlanRows = 37;
struct MeasuredPlans {
    int N, K;
    GemmPlan at[kPlanRows];
};
// The same for batched questions, M = 65 … 255 (entry i for M in (64 + 8 i, 72 + 8 i]), every
// configuration of the three kernels timed the same way on random weights and activations (two runs
// averaged); at M = 120 the hand-tuned rules below were already the fastest for all five shapes.
constexpr int kQRows = 24;
struct MeasuredQPlans {
    int N, K;
    GemmPlan at[kQRows];
};
const MeasuredQPlans kMeasuredQ[] = {
    // gate_up (the SiLU epilogue)
    {12288, 2048,
     {
         {P32, 1}, {P32, 1}, {P32, 1}, {P32, 1}, {W21h, 1}, {W21h, 1}, {W21h, 1}, {W21h, 1},
         {W31h, 1}, {W31h, 1}, {W31h, 1}, {W31h, 1}, {W31h, 1}, {W31h, 1}, {W31h, 1}, {W31h, 1},
         {W41, 1}, {P32, 1}, {P32, 1}, {P32, 1}, {W41h, 1}, {W41, 1}, {W41, 1}, {W41h, 1},
     }},
    // in_proj
    {8256, 2048,
     {
         {P21, 1}, {P21, 1}, {P21, 1}, {P21, 1}, {P31, 1}, {P31, 1}, {P31, 1}, {P31, 1},
         {P31, 1}, {P31, 1}, {W21h, 1}, {W21h, 1}, {W21h, 1}, {W21h, 1}, {W21h, 1}, {W21h, 1},
         {W31h, 1}, {W31h, 1}, {P31, 1}, {P22, 1}, {W31h, 1}, {P31, 1}, {W31h, 1}, {W31h, 1},
     }},
    // qkv
    {5120, 2048,
     {
         {P21, 1}, {P21, 1}, {P21, 1}, {P21, 1}, {P31, 1}, {P31, 1}, {P31, 1}, {P31, 1},
         {P31, 1}, {P31, 1}, {P41, 1}, {P21, 1}, {P41, 1}, {P41, 1}, {P41, 1}, {P21, 1},
         {P31, 1}, {P31, 1}, {P31, 1}, {P32, 1}, {P31, 1}, {P31, 1}, {P31, 1}, {W21h, 1},
     }},
    // out_proj and o_proj (split-K partials)
    {2048, 2048,
     {
         {P31, 4}, {P31, 4}, {P31, 4}, {P31, 4}, {P21, 2}, {P21, 2}, {P21, 2}, {P21, 2},
         {P31, 2}, {P31, 2}, {P31, 2}, {P31, 2}, {P31, 2}, {P31, 2}, {P31, 2}, {P31, 2},
         {P21, 2}, {P21, 2}, {P21, 2}, {P21, 2}, {P21, 2}, {P21, 2}, {P21, 2}, {P21, 2},
     }},
    // down (split-K partials)
    {2048, 6144,
     {
         {P31, 4}, {P31, 4}, {P31, 4}, {P31, 4}, {P41, 4}, {P41, 4}, {P41, 4}, {P41, 4},
         {P31, 4}, {P31, 4}, {P31, 4}, {P31, 4}, {P31, 4}, {P31, 4}, {P31, 4}, {P31, 4},
         {P41, 4}, {P41, 4}, {W21h, 4}, {W21h, 4}, {W21h, 4}, {W21h, 4}, {P41, 4}, {W21h, 4},
     }},
};
const MeasuredPlans kMeasured[] = {
    // gate_up (the SiLU epilogue)
    {12288, 2048,
     {
         {W41h, 1}, {W21, 1}, {W31, 1}, {W31, 1}, {W21, 1}, {W41, 1}, {W41, 1}, {W31, 1},
         {W31, 1}, {W21, 1}, {W31, 1}, {W31, 1}, {W41, 1}, {W31, 1}, {W31, 1}, {W31, 1},
         {W42, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W31, 1},
         {W41, 1}, {W41, 1}, {W41, 1}, {W41, 1}, {W41, 1}, {W41, 1}, {W41, 1}, {W41, 1},
         {W41, 1}, {W42, 1}, {W42, 1}, {W42, 1}, {W42, 1},
     }},
    // in_proj
    {8256, 2048,
     {
         {W31h, 1}, {W41h, 1}, {W41h, 1}, {W21h, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W21, 1},
         {W41, 1}, {W41, 1}, {W41, 1}, {W31, 1}, {W31, 1}, {W21, 1}, {W21, 1}, {W31, 1},
         {W31, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W42, 1}, {W42, 1},
         {W42, 1}, {W42, 1}, {W42, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W41, 1},
         {W42, 1}, {W42, 1}, {W42, 1}, {W42, 1}, {W42, 1},
     }},
    // qkv
    {5120, 2048,
     {
         {W21h, 1}, {W21h, 1}, {W21h, 1}, {W31h, 1}, {W31h, 1}, {W31h, 1}, {W41h, 1}, {W41h, 1},
         {W41h, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W21, 1},
         {W41, 1}, {W41, 1}, {W41, 1}, {W41, 1}, {W41, 1}, {W31, 1}, {W31, 1}, {W31, 1},
         {W31, 1}, {W41, 1}, {W41, 1}, {W41, 1}, {W41, 1}, {W41, 1}, {W41, 1}, {W41, 1},
         {W41, 1}, {W41, 1}, {W41, 1}, {W42, 1}, {W42, 1},
     }},
    // out_proj and o_proj (split-K partials)
    {2048, 2048,
     {
         {W21, 4}, {W21h, 2}, {W21h, 2}, {W21h, 2}, {W21h, 2}, {W31h, 2}, {W31h, 2}, {W31h, 2},
         {W31h, 2}, {W21h, 1}, {W21h, 1}, {W21h, 1}, {W21h, 1}, {W31h, 1}, {W31h, 1}, {W31h, 1},
         {W31h, 1}, {W31h, 1}, {W31h, 1}, {W31h, 1}, {W31h, 1}, {W21, 1}, {W21, 1}, {W21, 1},
         {W21, 1}, {W21, 1}, {W21, 1}, {W21, 1}, {W21, 1}, {W31, 1}, {W31, 1}, {W31, 1},
         {W31, 1}, {W31, 1}, {W31, 1}, {W31, 1}, {W31, 1},
     }},
    // down (split-K partials)
    {2048, 6144,
     {
         {W21h, 4}, {W31h, 4}, {W31h, 4}, {W21, 4}, {W21h, 2}, {W31h, 2}, {W31h, 2}, {W31h, 2},
         {W31h, 2}, {W41h, 2}, {W41h, 2}, {W41h, 2}, {W41h, 2}, {W31, 4}, {W31, 4}, {W31h, 1},
         {W31h, 1}, {W31h, 1}, {W31h, 1}, {W31h, 1}, {W31h, 1}, {W41h, 1}, {W41h, 1}, {W41h, 1},
         {W41h, 1}, {W41h, 1}, {W41h, 1}, {W41h, 1}, {W41h, 1}, {W31, 2}, {W31, 2}, {W31, 2},
         {W31, 2}, {W41, 2}, {W41, 2}, {W41, 2}, {W22, 2},
     }},
};

}  // namespace

int gemm_w4_configs() { return kNumCfgs; }

int gemm_w4_cfg(int M, bool exact) { return pick_cfg(M, exact); }

GemmPlan gemm_w4_plan(int M, int N, int K, bool exact, bool partial_ok, size_t max_part_elems) {
    GemmPlan p{pick_cfg(M, exact), 1};
    const bool wide_ok = K % 256 == 0, halves_ok = K % 512 == 0;
    auto fit = [&](GemmPlan q) {  // largest usable split <= q.ks
        const int steps = K / KSTEP;
        while (q.ks > 1 && (steps % q.ks || (size_t)q.ks * M * N > max_part_elems ||
                            (kCfgs[q.cfg].wide && (K / 64 / q.ks) % (4 * kCfgs[q.cfg].kh)) ||
                            (kCfgs[q.cfg].pipe && (steps / q.ks) % 4)))
            q.ks /= 2;
        return q;
    };
    if (!exact && M > 64 && M < 256)
        for (const MeasuredQPlans& t : kMeasuredQ)
            if (t.N == N && t.K == K) {
                const GemmPlan q = t.at[(M - 65) / 8];
                if (q.ks == 1 || partial_ok) return fit(q);
            }
    if (!exact && M >= 256 && M <= 256 + 64 * (kPlanRows - 1))
        for (const MeasuredPlans& t : kMeasured)
            if (t.N == N && t.K == K) {
                const GemmPlan q = t.at[(M - 193) / 64];
                if (q.ks == 1 || partial_ok) return fit(q);
            }
    if (!exact && wide_ok && M >= 256 && M <= 1024) {
        // Prefill-sized M; from a sweep of the 2B's shapes at M = 512 on MI355X (random data, tiled
        // weights): N = 12288 with the SiLU epilogue: (2,1) 33.2 us, (4,1) 34.5 us (3 runs each on
        // one box; 768 workgroups are 3 per CU where 384 are 1.5); N = 8256: (3,1) 24.8 us;
        // N = 5120: (3,1) with k halves 16.8 us; N = 2048: (2,1) with k halves and 2 splits 9.0 us
        // (K = 2048; 9.6 us without k halves, 3 runs each on one box),
        // (4,1) with 4 splits 18.8 us (K = 6144; (2,1) is 18.2 us alone but 22.5 us inside the
        // forward).
        // (3,1) with k halves holds one 512-thread workgroup per CU: only for grids of one round
        const bool one_round = (size_t)((N + 127) / 128) * ((M + 95) / 96) <= 256;
        if (N >= 10000) p.cfg = W21;
        else if (N >= 4000) p.cfg = halves_ok && one_round ? W31h : W31;
        else if (partial_ok && K > 3000) p = GemmPlan{W41, 4};
        else if (partial_ok) p = GemmPlan{halves_ok ? W21h : W21, 2};  // k halves: 9.04 vs 9.56 us
        else p.cfg = W21;
        return fit(p);
    }
    if (!exact && wide_ok && M > 1024) {
        // Long prefill, no K split (sweep at M = 1536 and 2048): gate_up (4,1) 106.9 us at 2048, (3,1)
        // 80.1 us at 1536; in_proj (3,1) 77.2 / 61.2 us; qkv (4,1) 51.9 / 35.3 us; N = 2048 (3,1)
        // with k halves where its grid is one round (43.2 us down, 17.6 us o at 1536), else (4,1)
        // (57.9 / 22.3 us at 2048).  The 16x16 (4,2) tiles take 26-50% longer at these sizes.
        const bool one_round = (size_t)((N + 127) / 128) * ((M + 95) / 96) <= 256;
        if (N >= 10000) p.cfg = M >= 1792 ? W41 : W31;
        else if (N >= 7000) p.cfg = W31;
        else if (N >= 4000) p.cfg = W41;
        else p.cfg = halves_ok && one_round ? W31h : W41;
        return p;
    }
    if (!exact && wide_ok && M > 64 && M < 256) {
        // Batched questions (M = 120), chosen inside the 2B's question forward (whole-forward A/B on
        // one box, one plan changed at a time; weights are cold there, unlike in a loop over one
        // GEMM): the 16x16 tiles with loads three steps ahead for in_proj (N = 8256) and qkv
        // (N = 5120), (3,1) (0.4 and 2 us per layer better than the 32x32 (2,1) with k halves and the
        // 16x16 (3,1)); out_proj / o_proj (2,1) with 2 splits (0.8 us per layer better than 16x16
        // (2,1) with 4); down (K = 6144) (4,1) with 4 splits (0.6 us better than 32x32 (2,1) with 8).
        // gate_up (N = 12288, SiLU) stays on 32x32 (2,1) with k halves: every 16x16 plan was 1-2 us
        // per layer slower there, though 5 us faster in a loop over the one GEMM.
        const bool pipe_ok = K % 512 == 0;
        if (!partial_ok) p.cfg = N >= 10000 || (N >= 7000 && !pipe_ok) ? (halves_ok ? W21h : W21) : pipe_ok ? P31 : T31;
        else if (N >= 10000) p = GemmPlan{W41, 2};
        else if (K > 3000) p = pipe_ok && (K / KSTEP) % 16 == 0 ? GemmPlan{P41, 4} : GemmPlan{W21, 8};
        else p = pipe_ok ? GemmPlan{P21, 2} : GemmPlan{T21, 4};
        return fit(p);
    }
    if (!exact && M > 64 && M < 256) p.cfg = partial_ok ? T41 : 4;
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
           (!c.wide || (steps / (ks * 2)) % (2 * c.kh) == 0) && (!c.pipe || (steps / (ks * 2)) % 4 == 0) &&
           (size_t)(ks * 2) * M * N <= max_part_elems)
        ks *= 2;
    return ks;
}

namespace {
// A GEMM launch; while Engine::profile times a step, the step's first GEMM records its own start
// and end (see KernelEvents).
void launch_gemm(GemmFn kern, dim3 grid, int threads, hipStream_t st, const f16* A, const uint32_t* W, const f16* S,
                 f16* Y, float* part, int M, int N, int K, int ks, bool tiled) {
    const int kt = ks << 1 | (tiled ? 1 : 0);
    KernelEvents* ke = kernel_events();
    if (ke && ke->launches == 0) {
        hipExtLaunchKernelGGL(kern, grid, dim3(threads), 0, st, ke->start, ke->stop, 0u, A, W, S, Y, part, M, N, K, kt);
        ke->launches++;
    } else {
        hipLaunchKernelGGL(kern, grid, dim3(threads), 0, st, A, W, S, Y, part, M, N, K, kt);
    }
}
}  // namespace

bool w4_tileable(int N, int K) { return N >= 32 && N % 32 == 0 && K >= 64 && K % 64 == 0; }

void gemm_w4(const f16* A, const uint32_t* W, const f16* S, f16* Y, float* part, int M, int N, int K, bool exact,
             int ks, hipStream_t st, int cfg, bool tiled) {
    SD_CHECK(M >= 1 && N >= 1 && K >= KSTEP && K % KSTEP == 0, "gemm_w4: need M, N >= 1 and K a multiple of 128");
    SD_CHECK(!tiled || w4_tileable(N, K), "gemm_w4: the tiled layout needs N a multiple of 32");
    const int ci = cfg >= 0 ? cfg : pick_cfg(M, exact);
    SD_CHECK(ci < kNumCfgs, "gemm_w4: bad configuration index");
    const Cfg& c = kCfgs[ci];
    SD_CHECK(c.exact == exact, "gemm_w4: configuration does not match the dequant mode");
    SD_CHECK(ks >= 1 && (K / KSTEP) % ks == 0, "gemm_w4: split count must divide the k steps");
    SD_CHECK(part || (Y && ks == 1), "gemm_w4: split-K writes partials and needs a partial buffer");
    SD_CHECK(!c.pipe || (K / KSTEP / ks) % 4 == 0, "gemm_w4: this configuration needs K / ks a multiple of 512");
    SD_CHECK(!c.wide || (K / 64 / ks) % (4 * c.kh) == 0,
             c.kh == 1 ? "gemm_w4: this configuration needs K / ks a multiple of 256"
                       : "gemm_w4: this configuration needs K / ks a multiple of 256 per k half");
    const int bm = c.mt * 16, bn = 4 * c.nt * 16;
    dim3 grid((N + bn - 1) / bn, (M + bm - 1) / bm, ks);
    launch_gemm(part ? c.part_out : c.f16_out, grid, 256 * c.kh, st, A, W, S, Y, part, M, N, K, ks, tiled);
    launched("gemm_w4");
}

bool gemm_w4_has_silu(int cfg) { return cfg >= 0 && cfg < kNumCfgs && kCfgs[cfg].silu_out != nullptr; }

void gemm_w4_silu(const f16* A, const uint32_t* W, const f16* S, f16* mid, int M, int N, int K, hipStream_t st,
                  int cfg, bool tiled) {
    SD_CHECK(cfg >= 0 && cfg < kNumCfgs && kCfgs[cfg].silu_out, "gemm_w4_silu: no SiLU epilogue in this configuration");
    const Cfg& c = kCfgs[cfg];
    SD_CHECK(M >= 1 && N >= 32 && N % 32 == 0 && K % ((c.pipe ? 512 : 256) * c.kh) == 0,
             c.pipe ? "gemm_w4_silu: need N a multiple of 32 and K of 512"
                    : "gemm_w4_silu: need N a multiple of 32 and K of 256 per k half");
    const int bm = c.mt * 16, bn = 4 * c.nt * 16;
    dim3 grid((N + bn - 1) / bn, (M + bm - 1) / bm, 1);
    launch_gemm(c.silu_out, grid, 256 * c.kh, st, A, W, S, mid, (float*)nullptr, M, N, K, 1, tiled);
    launched("gemm_w4_silu");
}

void tile_w4(uint32_t* W, f16* S, int N, int K, void* tmp, hipStream_t st) {
    SD_CHECK(w4_tileable(N, K), "tile_w4: need N a multiple of 32 and K of 64");
    const int KB = K / 32;
    const size_t blocks = (size_t)N * KB;
    u32x4* tw = static_cast<u32x4*>(tmp);
    f16* ts = reinterpret_cast<f16*>(tw + blocks);
    hipLaunchKernelGGL(k_tile_w4, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<const u32x4*>(W), S, tw, ts, N, KB);
    launched("tile_w4");
    SD_HIP(hipMemcpyAsync(W, tw, blocks * 16, hipMemcpyDeviceToDevice, st));
    SD_HIP(hipMemcpyAsync(S, ts, blocks * 2, hipMemcpyDeviceToDevice, st));
}

void interleave_gate_up(uint32_t* W, f16* S, int N, int K, void* tmp, hipStream_t st) {
    SD_CHECK(N % 32 == 0 && K % 32 == 0, "interleave_gate_up: need N a multiple of 32");
    const int KB = K / 32;
    u32x4* tw = static_cast<u32x4*>(tmp);
    f16* ts = reinterpret_cast<f16*>(tw + (size_t)N * KB);
    hipLaunchKernelGGL(k_interleave_gate_up, dim3(N), dim3(256), 0, st, reinterpret_cast<const u32x4*>(W), S, tw, ts,
                       N, KB);
    launched("interleave_gate_up");
    SD_HIP(hipMemcpyAsync(W, tw, (size_t)N * KB * 16, hipMemcpyDeviceToDevice, st));
    SD_HIP(hipMemcpyAsync(S, ts, (size_t)N * KB * 2, hipMemcpyDeviceToDevice, st));
}

void repack_w4(uint32_t* W, size_t words, hipStream_t st) {
    if (!words) return;
    hipLaunchKernelGGL(k_repack_w4, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, st, W, words);
    launched("repack_w4");
}

void reduce_partials(const float* part, int ks, size_t n, f16* Y, hipStream_t st) {
    const size_t threads = (n + 3) / 4;
    hipLaunchKernelGGL(k_reduce_partials, dim3((threads + 255) / 256), dim3(256), 0, st, part, ks, n, Y);
    launched("reduce_partials");
}

}  // namespace sd
