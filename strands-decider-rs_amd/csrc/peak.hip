// Achievable-peak microbenchmarks on gfx950 (libsdpeak.so; not part of the engine).  The roofline
// fractions the benchmark reports are against MI355X's published peaks (2.5 PFLOP/s dense f16 MFMA,
// 8 TB/s HBM); these loops measure what this chip sustains for the same instruction mix, so that a
// kernel's fraction can also be stated against an achievable ceiling:
//  * k_mfma_loop: v_mfma_f32_32x32x16_f16 (the prefill GEMM's instruction) from register operands,
//    NACC independent accumulator chains per wave, no memory traffic;
//  * k_gemm_mix: the prefill GEMM's inner loop without its memory traffic: per 16-k slice one
//    int4 word dequantized exactly as the GEMM does (v_and_or_b32 nibble pairs, packed f16 subtract
//    or fma, times the scale), MT2 A fragments read from LDS, and MT2 MFMAs fed by them (the GEMM's
//    (2,1) tiles: 6.5 dequant VALU instructions per MFMA), with the GEMM's software pipeline and
//    issue pins.  The word changes every slice (xor with the loop counter, one more VALU
//    instruction), so nothing can be hoisted out of the loop;
//  * k_hbm_read / k_hbm_copy: streaming 16-byte loads (and stores) over a buffer much larger than
//    the 256 MB last-level cache.
// Every workgroup stamps the shader clock (s_memtime) and the 100 MHz constant clock (s_memrealtime)
// at its start and end, which gives the clock the loop actually ran at.
#include "../../include/sdpeak.h"
#include "common.h"
#include "device.h"

namespace sd {
namespace {

struct Stamp {
    uint64_t t0, t1, r0, r1;  // shader clock and 100 MHz clock at the workgroup's start and end
};

__device__ __forceinline__ void stamp_begin(Stamp* st) {
    if (threadIdx.x == 0) {
        st[blockIdx.x].t0 = __builtin_amdgcn_s_memtime();
        st[blockIdx.x].r0 = __builtin_amdgcn_s_memrealtime();
    }
}
__device__ __forceinline__ void stamp_end(Stamp* st) {
    __syncthreads();
    if (threadIdx.x == 0) {
        st[blockIdx.x].t1 = __builtin_amdgcn_s_memtime();
        st[blockIdx.x].r1 = __builtin_amdgcn_s_memrealtime();
    }
}

// RAND: four operand sets per lane of random f16 (random signs and mantissas, magnitudes 2^-3 to 1,
// like an RMSNorm output's) taken in turn, so that consecutive MFMAs see different bits as they do
// in a GEMM; otherwise one set of 3-bit patterns for every MFMA (few bits switch: the instruction
// rate at the clock such operands allow).
template <int NACC, bool RAND>
__global__ __launch_bounds__(256) void k_mfma_loop(int iters, const u32x4* __restrict__ rnd, float* __restrict__ sink,
                                                   Stamp* __restrict__ st) {
    stamp_begin(st);
    const int lane = threadIdx.x & 63;
    f16x8 a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        if constexpr (RAND) {
            a[u] = __builtin_bit_cast(f16x8, rnd[(threadIdx.x * 8 + 2 * u) & 2047]);
            b[u] = __builtin_bit_cast(f16x8, rnd[(threadIdx.x * 8 + 2 * u + 1) & 2047]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                a[u][e] = (f16)(0.001f * (float)((lane + e) & 7));
                b[u][e] = (f16)(0.002f * (float)((lane * 3 + e) & 7));
            }
        }
    }
    f32x16 acc[NACC];
#pragma unroll
    for (int n = 0; n < NACC; n++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[n][i] = 0.f;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int n = 0; n < NACC; n++) acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[u], b[u], acc[n], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int n = 0; n < NACC; n++)
#pragma unroll
        for (int i = 0; i < 16; i++) s += acc[n][i];
    sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
    stamp_end(st);
}

// RAND: the A tile in LDS holds random f16 as k_mfma_loop's, and each k slice's scale is its own
// random f16 of a trained model's magnitude; otherwise a patterned A tile and one scale.  The
// weight words are random either way (the nibbles are what the dequant sees).
template <int MT2, bool RAND>
__global__ __launch_bounds__(256) void k_gemm_mix(int iters, const uint32_t* __restrict__ words, const u32x4* __restrict__ rnd,
                                                  float* __restrict__ sink, Stamp* __restrict__ st) {
    stamp_begin(st);
    __shared__ __attribute__((aligned(16))) uint8_t lds[MT2 * 4096];
    const int tid = threadIdx.x, lane = tid & 63, r = lane & 31, g = lane >> 5;
    if constexpr (RAND) {
        for (int i = tid; i < MT2 * 256; i += 256) reinterpret_cast<u32x4*>(lds)[i] = rnd[i & 2047];
    } else {
        for (int i = tid; i < MT2 * 1024; i += 256) reinterpret_cast<uint32_t*>(lds)[i] = 0x1C001C00u ^ (uint32_t)(i & 0x3FF);
    }
    __syncthreads();
    uint32_t w[4];
#pragma unroll
    for (int s = 0; s < 4; s++) w[s] = words[(lane * 4 + s) & 255];
    f16x2 scs[4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const f16 v = RAND ? __builtin_bit_cast(f16, (uint16_t)(0x2000u | (words[(lane * 4 + s + 1) & 255] & 0x3FFu)))
                           : (f16)0.01f;
        scs[s] = f16x2{v, v};
    }
    // the GEMM's fragment offsets: row r, k-chunk 4g + s, XOR-swizzled by row pair
    uint32_t foff[4];
#pragma unroll
    for (int s = 0; s < 4; s++) foff[s] = r * 128 + (((4 * g + s) ^ ((r >> 1) & 7)) << 4);
    f32x16 acc[MT2];
#pragma unroll
    for (int a = 0; a < MT2; a++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[a][i] = 0.f;
    // the GEMM's software pipeline and issue pins (k_gemm_w4m): slice s + 1's fragments and weights
    // are produced while slice s's MFMAs run, one MFMA then its share of the dequant VALU
    // instructions then a fragment read
    constexpr int VPER = (13 + MT2 - 1) / MT2;
    auto deq = [&](uint32_t word, int s) {
        f16x2 p0, p1, p2, p3;
        nib_pairs(word, p0, p1, p2, p3);
        const f16x2 sc2 = scs[s];
        return cat4(p0 * sc2, p1 * sc2, p2 * sc2, p3 * sc2);
    };
    auto frag = [&](int s, f16x8* af) {
#pragma unroll
        for (int a = 0; a < MT2; a++) af[a] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(lds + a * 4096 + foff[s]));
    };
    f16x8 bf0 = deq(w[0], 0);
    for (int it = 0; it < iters; it++) {
        f16x8 af[2][MT2], bf[2];
        bf[0] = bf0;
        frag(0, af[0]);
        __builtin_amdgcn_sched_group_barrier(0x100, MT2, 0);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int cu = s & 1, nx = cu ^ 1;
            if (s < 3) {
                frag(s + 1, af[nx]);
                bf[nx] = deq(w[s + 1] ^ (uint32_t)it, s + 1);
            } else {
                bf0 = deq(w[0] ^ (uint32_t)(it + 1), 0);
            }
#pragma unroll
            for (int a = 0; a < MT2; a++) acc[a] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[cu], af[cu][a], acc[a], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < MT2; j++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);     // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, VPER, 0);  // VALU
                if (s < 3) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // a fragment read
            }
        }
    }
    float s = 0.f;
#pragma unroll
    for (int a = 0; a < MT2; a++)
#pragma unroll
        for (int i = 0; i < 16; i++) s += acc[a][i];
    sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
    stamp_end(st);
}

// Grid-stride streaming: 4 independent 16-byte loads in flight per thread and round.
__global__ __launch_bounds__(256) void k_hbm_read(const u32x4* __restrict__ src, size_t n16, uint32_t* __restrict__ sink,
                                                  Stamp* __restrict__ st) {
    stamp_begin(st);
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    u32x4 x = {0u, 0u, 0u, 0u};
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u32x4 v0 = __builtin_nontemporal_load(src + i), v1 = __builtin_nontemporal_load(src + i + stride);
        const u32x4 v2 = __builtin_nontemporal_load(src + i + 2 * stride), v3 = __builtin_nontemporal_load(src + i + 3 * stride);
        x ^= v0 ^ v1 ^ v2 ^ v3;
    }
    for (; i < n16; i += stride) x ^= src[i];
    sink[blockIdx.x * blockDim.x + threadIdx.x] = x[0] ^ x[1] ^ x[2] ^ x[3];
    stamp_end(st);
}

__global__ __launch_bounds__(256) void k_hbm_copy(const u32x4* __restrict__ src, u32x4* __restrict__ dst, size_t n16,
                                                  Stamp* __restrict__ st) {
    stamp_begin(st);
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u32x4 v0 = __builtin_nontemporal_load(src + i), v1 = __builtin_nontemporal_load(src + i + stride);
        const u32x4 v2 = __builtin_nontemporal_load(src + i + 2 * stride), v3 = __builtin_nontemporal_load(src + i + 3 * stride);
        __builtin_nontemporal_store(v0, dst + i);
        __builtin_nontemporal_store(v1, dst + i + stride);
        __builtin_nontemporal_store(v2, dst + i + 2 * stride);
        __builtin_nontemporal_store(v3, dst + i + 3 * stride);
    }
    for (; i < n16; i += stride) dst[i] = src[i];
    stamp_end(st);
}

void put_err(char* err, size_t errlen, const char* msg) {
    if (!err || errlen == 0) return;
    size_t i = 0;
    for (; msg[i] && i + 1 < errlen; i++) err[i] = msg[i];
    err[i] = '\0';
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

// Number of compute units of the current device.
int device_cus() {
    int dev = 0, cus = 0;
    SD_HIP(hipGetDevice(&dev));
    SD_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    return cus;
}

// Launches `launches` back-to-back launches of `launch(stamps)` between two events; fills the
// wall-clock ms of all launches and the mean shader clock (GHz) of the last launch's workgroups.
template <class L>
void timed(int launches, int blocks, hipStream_t s, L&& launch, double& ms, double& ghz) {
    Stamp* st = nullptr;
    SD_HIP(hipMalloc(&st, sizeof(Stamp) * blocks));
    hipEvent_t e0 = nullptr, e1 = nullptr;
    try {
        SD_HIP(hipEventCreate(&e0));
        SD_HIP(hipEventCreate(&e1));
        launch(st);  // warm-up (code load, first-touch)
        SD_HIP(hipEventRecord(e0, s));
        for (int i = 0; i < launches; i++) launch(st);
        SD_HIP(hipEventRecord(e1, s));
        SD_HIP(hipEventSynchronize(e1));
        float f = 0.f;
        SD_HIP(hipEventElapsedTime(&f, e0, e1));
        ms = f;
        std::vector<Stamp> h(blocks);
        SD_HIP(hipMemcpy(h.data(), st, sizeof(Stamp) * blocks, hipMemcpyDeviceToHost));
        double sum = 0.0;
        int n = 0;
        for (const Stamp& x : h)
            if (x.r1 > x.r0) {
                sum += (double)(x.t1 - x.t0) / (double)(x.r1 - x.r0) * 0.1;  // 100 MHz constant clock
                n++;
            }
        ghz = n ? sum / n : 0.0;
    } catch (...) {
        if (e0) (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
        (void)hipFree(st);
        throw;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    SD_HIP(hipFree(st));
}

}  // namespace
}  // namespace sd

extern "C" int sd_peak_mfma(int variant, int wg_per_cu, int iters, int launches, void* stream, double* out, char* err,
                            size_t errlen) {
    return sd::guarded(err, errlen, [&] {
        if (!out) throw sd::Error("sd_peak_mfma: null output");
        if (variant < 0 || variant > 5) throw sd::Error("sd_peak_mfma: variant must be 0 to 5");
        if (wg_per_cu < 1 || wg_per_cu > 4 || iters < 1 || launches < 1)
            throw sd::Error("sd_peak_mfma: 1 to 4 workgroups per CU, iters and launches >= 1");
        const hipStream_t s = static_cast<hipStream_t>(stream);
        const int cus = sd::device_cus(), blocks = cus * wg_per_cu;
        float* sink = nullptr;
        uint32_t* words = nullptr;
        sd::u32x4* rnd = nullptr;
        SD_HIP(hipMalloc(&sink, (size_t)blocks * 256 * 4));
        double ms = 0.0, ghz = 0.0;
        try {
            SD_HIP(hipMalloc(&words, 256 * 4));
            SD_HIP(hipMalloc(&rnd, 2048 * 16));
            std::vector<uint32_t> hw(256), hr(2048 * 4);
            uint32_t x = 0x2545F491u;  // xorshift32
            auto next = [&] {
                x ^= x << 13;
                x ^= x >> 17;
                x ^= x << 5;
                return x;
            };
            for (uint32_t& v : hw) v = next();
            // f16 pairs: random sign and mantissa, exponent field 12 to 15 (2^-3 <= |v| < 1)
            for (uint32_t& v : hr) {
                const uint32_t b = next();
                const uint32_t lo = (b & 0x83FFu) | ((12u + ((b >> 10) & 3u)) << 10);
                const uint32_t c = next();
                const uint32_t hi = (c & 0x83FFu) | ((12u + ((c >> 10) & 3u)) << 10);
                v = lo | hi << 16;
            }
            SD_HIP(hipMemcpy(words, hw.data(), 256 * 4, hipMemcpyHostToDevice));
            SD_HIP(hipMemcpy(rnd, hr.data(), hr.size() * 4, hipMemcpyHostToDevice));
            sd::timed(launches, blocks, s, [&](void* st) {
                auto* stp = static_cast<sd::Stamp*>(st);
                if (variant == 0)
                    hipLaunchKernelGGL((sd::k_mfma_loop<4, false>), dim3(blocks), dim3(256), 0, s, iters, rnd, sink, stp);
                else if (variant == 1)
                    hipLaunchKernelGGL((sd::k_gemm_mix<2, false>), dim3(blocks), dim3(256), 0, s, iters, words, rnd, sink, stp);
                else if (variant == 2)
                    hipLaunchKernelGGL((sd::k_gemm_mix<4, false>), dim3(blocks), dim3(256), 0, s, iters, words, rnd, sink, stp);
                else if (variant == 3)
                    hipLaunchKernelGGL((sd::k_mfma_loop<4, true>), dim3(blocks), dim3(256), 0, s, iters, rnd, sink, stp);
                else if (variant == 4)
                    hipLaunchKernelGGL((sd::k_gemm_mix<2, true>), dim3(blocks), dim3(256), 0, s, iters, words, rnd, sink, stp);
                else
                    hipLaunchKernelGGL((sd::k_gemm_mix<4, true>), dim3(blocks), dim3(256), 0, s, iters, words, rnd, sink, stp);
                SD_HIP(hipGetLastError());
            }, ms, ghz);
        } catch (...) {
            (void)hipFree(sink);
            (void)hipFree(words);
            (void)hipFree(rnd);
            throw;
        }
        SD_HIP(hipFree(sink));
        SD_HIP(hipFree(words));
        SD_HIP(hipFree(rnd));
        const int v3 = variant % 3;
        const int mfma_per_wave_iter = v3 == 0 ? 4 * 4 : v3 == 1 ? 4 * 2 : 4 * 4;
        const double flops = (double)launches * blocks * 4 * iters * mfma_per_wave_iter * 32768.0;
        out[0] = ms;
        out[1] = flops / (ms * 1e-3) / 1e12;
        out[2] = ghz;
        out[3] = cus;
    });
}

extern "C" int sd_peak_hbm(int variant, size_t bytes, int launches, void* stream, double* out, char* err, size_t errlen) {
    return sd::guarded(err, errlen, [&] {
        if (!out) throw sd::Error("sd_peak_hbm: null output");
        if (variant < 0 || variant > 1) throw sd::Error("sd_peak_hbm: variant must be 0 (read) or 1 (copy)");
        if (bytes < (size_t(1) << 20) || bytes % 16 || launches < 1)
            throw sd::Error("sd_peak_hbm: at least 1 MiB, a multiple of 16 bytes, launches >= 1");
        const hipStream_t s = static_cast<hipStream_t>(stream);
        const int cus = sd::device_cus(), blocks = cus * 8;
        const size_t n16 = bytes / 16;
        void *src = nullptr, *dst = nullptr, *sink = nullptr;
        double ms = 0.0, ghz = 0.0;
        try {
            SD_HIP(hipMalloc(&src, bytes));
            SD_HIP(hipMemsetAsync(src, 0x5A, bytes, s));
            if (variant == 1) SD_HIP(hipMalloc(&dst, bytes));
            SD_HIP(hipMalloc(&sink, (size_t)blocks * 256 * 4));
            sd::timed(launches, blocks, s, [&](void* st) {
                auto* stp = static_cast<sd::Stamp*>(st);
                if (variant == 0)
                    hipLaunchKernelGGL(sd::k_hbm_read, dim3(blocks), dim3(256), 0, s, static_cast<const sd::u32x4*>(src), n16,
                                       static_cast<uint32_t*>(sink), stp);
                else
                    hipLaunchKernelGGL(sd::k_hbm_copy, dim3(blocks), dim3(256), 0, s, static_cast<const sd::u32x4*>(src),
                                       static_cast<sd::u32x4*>(dst), n16, stp);
                SD_HIP(hipGetLastError());
            }, ms, ghz);
        } catch (...) {
            (void)hipFree(src);
            (void)hipFree(dst);
            (void)hipFree(sink);
            throw;
        }
        SD_HIP(hipFree(src));
        if (dst) SD_HIP(hipFree(dst));
        SD_HIP(hipFree(sink));
        const double moved = (double)launches * (double)bytes * (variant == 1 ? 2.0 : 1.0);
        out[0] = ms;
        out[1] = moved / (ms * 1e-3) / 1e9;  // GB/s
        out[2] = ghz;
        out[3] = cus;
    });
}
