// Row-wise and elementwise kernels: embedding gather, residual add + RMSNorm, SiLU gate,
// adapter bias, and a fill used instead of hipMemsetAsync (safe inside captured graphs).
#include <algorithm>

#include "common.h"
#include "device.h"

namespace sd {
namespace {

// Quant code of element e of block `blk` (src/kernels.rs:63-70).
__device__ __forceinline__ uint32_t qcode(const uint32_t* __restrict__ Q, size_t blk, int e, int bits) {
    if (bits == 4) return (Q[blk * 4 + (e >> 3)] >> (4 * (e & 7))) & 15u;
    uint32_t lo = (Q[blk * bits + (e >> 4)] >> (2 * (e & 15))) & 3u;
    if (bits == 3) lo |= ((Q[blk * 3 + 2] >> e) & 1u) << 2;
    return lo;
}

// x[t, :] = dequantized row ids[t] (src/kernels.rs:63-89).  One thread per 8 consecutive elements
// (a quarter of a 32-element block): two 16-byte stores, so that a wave writes 2 KiB of a row.
__global__ __launch_bounds__(256) void k_embed(const uint32_t* __restrict__ ids, int L,
                                               const uint32_t* __restrict__ Q, const f16* __restrict__ S,
                                               const f16* __restrict__ Bi, int d, int bits, int group, int asym,
                                               float* __restrict__ x) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;  // 8-element part of the row
    const int nb = d >> 5, b = i >> 2, e0 = 8 * (i & 3);
    if (t >= L || b >= nb) return;
    const size_t blk = (size_t)ids[t] * nb + b;
    const size_t gi = group == 32 ? blk : blk / (size_t)(group >> 5);
    const float sc = (float)S[gi];
    const float bi = asym ? (float)Bi[gi] : 0.f;
    const float off = (float)(1 << (bits - 1));
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const float q = (float)qcode(Q, blk, e0 + u, bits);
        v[u] = asym ? q * sc + bi : (q - off) * sc;
    }
    float4* out = reinterpret_cast<float4*>(x + (size_t)t * d + b * 32 + e0);
    out[0] = float4{v[0], v[1], v[2], v[3]};
    out[1] = float4{v[4], v[5], v[6], v[7]};
}

// One workgroup (256 threads) per output row; D = d / 256 values per thread.
// The sublayer output y is f16 rows, or ks f32 partial slots whose slot-order sum rounded to f16
// is that same f16 value.
template <int D, int KS>
__global__ __launch_bounds__(256) void k_add_norm(float* __restrict__ x, const f16* __restrict__ y,
                                                  const float* __restrict__ yp, size_t slot,
                                                  const float* __restrict__ w, const uint32_t* __restrict__ rows,
                                                  f16* __restrict__ h16, float* __restrict__ h32) {
    constexpr int d = D * 256;
    // D % 4 == 0: thread t takes the D consecutive elements [D t, D t + D) with 16-byte accesses;
    // otherwise element c = t + 256 i
    constexpr bool VEC = D % 4 == 0;
    __shared__ float red[4];
    const int r = blockIdx.x;
    const size_t row = rows ? rows[r] : (size_t)r;
    float* xr = x + row * d;
    auto col = [&](int i) { return VEC ? (int)threadIdx.x * D + i : (int)threadIdx.x + 256 * i; };
    float v[D], wv[D];
    float part[D][KS > 0 ? KS : 1];
    // issue every load of the row (and the norm weights) before using any
    if constexpr (VEC) {
#pragma unroll
        for (int i = 0; i < D; i += 4) {
            const int c = col(i);
            const float4 x4 = *reinterpret_cast<const float4*>(xr + c);
            const float4 w4 = *reinterpret_cast<const float4*>(w + c);
            v[i] = x4.x, v[i + 1] = x4.y, v[i + 2] = x4.z, v[i + 3] = x4.w;
            wv[i] = w4.x, wv[i + 1] = w4.y, wv[i + 2] = w4.z, wv[i + 3] = w4.w;
            if constexpr (KS > 0) {
#pragma unroll
                for (int z = 0; z < KS; z++) {
                    const float4 p4 = *reinterpret_cast<const float4*>(yp + z * slot + row * d + c);
                    part[i][z] = p4.x, part[i + 1][z] = p4.y, part[i + 2][z] = p4.z, part[i + 3][z] = p4.w;
                }
            } else {
#pragma unroll
                for (int u = 0; u < 4; u++) part[i + u][0] = y ? (float)y[row * d + c + u] : 0.f;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < D; i++) {
            const int c = col(i);
            v[i] = xr[c];
            wv[i] = w[c];
            if constexpr (KS > 0) {
#pragma unroll
                for (int z = 0; z < KS; z++) part[i][z] = yp[z * slot + row * d + c];
            } else {
                part[i][0] = y ? (float)y[row * d + c] : 0.f;
            }
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < D; i++) {
        float a = v[i];
        if constexpr (KS > 0) {
            float s = part[i][0];
#pragma unroll
            for (int z = 1; z < KS; z++) s += part[i][z];
            a += (float)(f16)s;
        } else if (y) {
            a += part[i][0];
        }
        v[i] = a;
        ss += a * a;
    }
    if (KS > 0 || y) {
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < D; i += 4)
                *reinterpret_cast<float4*>(xr + col(i)) = float4{v[i], v[i + 1], v[i + 2], v[i + 3]};
        } else {
#pragma unroll
            for (int i = 0; i < D; i++) xr[col(i)] = v[i];
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    lds_barrier();  // not __syncthreads, which would also wait for the x stores above
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / sqrtf(tot / (float)d + 1e-6f);
    if constexpr (VEC) {
#pragma unroll
        for (int i = 0; i < D; i += 4) {
            const int c = col(i);
            const float o0 = v[i] * inv * wv[i], o1 = v[i + 1] * inv * wv[i + 1], o2 = v[i + 2] * inv * wv[i + 2],
                        o3 = v[i + 3] * inv * wv[i + 3];
            if (h16) {
                const f16x4 o4 = {(f16)o0, (f16)o1, (f16)o2, (f16)o3};
                *reinterpret_cast<f16x4*>(h16 + (size_t)r * d + c) = o4;
            } else {
                *reinterpret_cast<float4*>(h32 + (size_t)r * d + c) = float4{o0, o1, o2, o3};
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < D; i++) {
            const int c = col(i);
            const float o = v[i] * inv * wv[i];
            if (h16) h16[(size_t)r * d + c] = (f16)o;
            else h32[(size_t)r * d + c] = o;
        }
    }
}

// mid[t, j] = f16(silu(g) * u), big[t] = [g | u] (src/kernels.rs:123-135).  8 values per thread.
// With KS > 0 the gate_up output arrives as KS f32 split-K slots of [L][2I]; their slot-order
// sum rounded to f16 is the f16 value the reference stores in `big`.  `il`: the engine's gate_up
// weights have their rows interleaved in groups of 16 (interleave_gate_up), so gate j sits at
// column 32 (j / 16) + j % 16 and up j 16 columns further.
template <int KS>
__global__ void k_silu_mul(const f16* __restrict__ big, const float* __restrict__ part, int L, int I, int il,
                           f16* __restrict__ mid) {
    const size_t i8 = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (i8 >= (size_t)L * I) return;
    const size_t t = i8 / I, j = i8 % I;
    const size_t gc = il ? (j >> 4) * 32 + (j & 15) : j, uc = il ? gc + 16 : I + j;
    float gv[8], uv[8];
    if constexpr (KS == 0) {
        const f16x8 g8 = *reinterpret_cast<const f16x8*>(big + t * 2 * I + gc);
        const f16x8 u8 = *reinterpret_cast<const f16x8*>(big + t * 2 * I + uc);
#pragma unroll
        for (int e = 0; e < 8; e++) gv[e] = (float)g8[e], uv[e] = (float)u8[e];
    } else {
        const size_t slot = (size_t)L * 2 * I;
        float4 g4[KS][2], u4[KS][2];
#pragma unroll
        for (int z = 0; z < KS; z++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                g4[z][h] = *reinterpret_cast<const float4*>(part + z * slot + t * 2 * I + gc + 4 * h);
                u4[z][h] = *reinterpret_cast<const float4*>(part + z * slot + t * 2 * I + uc + 4 * h);
            }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float4 gs = g4[0][h], us = u4[0][h];
#pragma unroll
            for (int z = 1; z < KS; z++) {
                gs.x += g4[z][h].x, gs.y += g4[z][h].y, gs.z += g4[z][h].z, gs.w += g4[z][h].w;
                us.x += u4[z][h].x, us.y += u4[z][h].y, us.z += u4[z][h].z, us.w += u4[z][h].w;
            }
            gv[4 * h] = (float)(f16)gs.x, gv[4 * h + 1] = (float)(f16)gs.y, gv[4 * h + 2] = (float)(f16)gs.z, gv[4 * h + 3] = (float)(f16)gs.w;
            uv[4 * h] = (float)(f16)us.x, uv[4 * h + 1] = (float)(f16)us.y, uv[4 * h + 2] = (float)(f16)us.z, uv[4 * h + 3] = (float)(f16)us.w;
        }
    }
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = (f16)silu_mul(gv[e], uv[e]);
    *reinterpret_cast<f16x8*>(mid + i8) = o;
}

__global__ void k_add_bias(f16* __restrict__ y, size_t n, int N, const float* __restrict__ c) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = (f16)((float)y[i] + c[i % N]);
}

struct U32x8 {
    uint32_t v[8];
};
__global__ void k_set_u32x8(uint32_t* __restrict__ p, U32x8 a) {
    if (threadIdx.x < 8) p[threadIdx.x] = a.v[threadIdx.x];
}

__global__ void k_fill_u32(uint32_t* __restrict__ p, size_t n, uint32_t v) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

}  // namespace

void embed(const uint32_t* ids, int L, const uint32_t* Q, const f16* S, const f16* Bi, int d, int bits, int group,
           bool asym, float* x, hipStream_t st) {
    SD_CHECK(d % 32 == 0 && (bits == 2 || bits == 3 || bits == 4) && group % 32 == 0 && group > 0,
             "embed: unsupported format");
    const int parts = d / 8;  // 8-element parts per row
    hipLaunchKernelGGL(k_embed, dim3((parts + 255) / 256, L), dim3(256), 0, st, ids, L, Q, S, Bi, d, bits, group,
                       (int)asym, x);
    launched("embed");
}

void add_norm(float* x, const YIn& y, const float* w, int d, const uint32_t* rows, int nrows, f16* h16, float* h32,
              hipStream_t st) {
    if (nrows == 0) return;
    const int ks = y.yp ? y.ks : 0;
    SD_CHECK(ks == 0 || ks == 1 || ks == 2 || ks == 4 || ks == 8, "add_norm: unsupported partial count");
    bool done = false;
#define SD_CASE(D, KS)                                                                                            \
    if (!done && d == D * 256 && ks == KS) {                                                                      \
        hipLaunchKernelGGL((k_add_norm<D, KS>), dim3(nrows), dim3(256), 0, st, x, y.y16, y.yp, y.slot, w, rows, h16, \
                           h32);                                                                                  \
        done = true;                                                                                              \
    }
#define SD_KS(D) SD_CASE(D, 0) SD_CASE(D, 1) SD_CASE(D, 2) SD_CASE(D, 4) SD_CASE(D, 8)
    SD_KS(1) SD_KS(2) SD_KS(3) SD_KS(4) SD_KS(6) SD_KS(8) SD_KS(10) SD_KS(12) SD_KS(16)
#undef SD_KS
#undef SD_CASE
    if (!done) throw Error("add_norm: hidden size " + std::to_string(d) + " is not supported");
    launched("add_norm");
}

// dst0 row r = src0 row rows[r] (bytes0 per row), and the same for src1/dst1: block (r, which)
// copies one row in 16-byte pieces
__global__ __launch_bounds__(256) void k_gather_rows2(const uint8_t* __restrict__ s0, uint8_t* __restrict__ d0,
                                                      uint32_t b0, const uint8_t* __restrict__ s1,
                                                      uint8_t* __restrict__ d1, uint32_t b1,
                                                      const uint32_t* __restrict__ rows) {
    const bool second = blockIdx.y != 0;
    const uint8_t* const src = second ? s1 : s0;
    uint8_t* const dst = second ? d1 : d0;
    const uint32_t b = second ? b1 : b0;
    const size_t r = blockIdx.x, row = rows[r];
    for (uint32_t i = threadIdx.x * 16u; i < b; i += 256u * 16u)
        *reinterpret_cast<u32x4*>(dst + r * b + i) = *reinterpret_cast<const u32x4*>(src + row * b + i);
}

void gather_rows2(const void* s0, void* d0, size_t bytes0, const void* s1, void* d1, size_t bytes1, const uint32_t* rows,
                  int n, hipStream_t st) {
    SD_CHECK(bytes0 % 16 == 0 && bytes1 % 16 == 0, "gather_rows2: rows must be multiples of 16 bytes");
    if (n == 0) return;
    hipLaunchKernelGGL(k_gather_rows2, dim3(n, 2), dim3(256), 0, st, static_cast<const uint8_t*>(s0),
                       static_cast<uint8_t*>(d0), (uint32_t)bytes0, static_cast<const uint8_t*>(s1), static_cast<uint8_t*>(d1),
                       (uint32_t)bytes1, rows);
    launched("gather");
}

void silu_mul(const f16* big, const float* part, int ks, int L, int I, bool il, f16* mid, hipStream_t st) {
    SD_CHECK(I % 8 == 0, "silu_mul: intermediate size must be a multiple of 8");
    SD_CHECK(!il || I % 16 == 0, "silu_mul: interleaved gate/up needs I a multiple of 16");
    const size_t n8 = (size_t)L * I / 8;
    const dim3 grid((n8 + 255) / 256);
    const int k = part ? ks : 0;
    switch (k) {
        case 0: hipLaunchKernelGGL(k_silu_mul<0>, grid, dim3(256), 0, st, big, part, L, I, il, mid); break;
        case 1: hipLaunchKernelGGL(k_silu_mul<1>, grid, dim3(256), 0, st, big, part, L, I, il, mid); break;
        case 2: hipLaunchKernelGGL(k_silu_mul<2>, grid, dim3(256), 0, st, big, part, L, I, il, mid); break;
        case 4: hipLaunchKernelGGL(k_silu_mul<4>, grid, dim3(256), 0, st, big, part, L, I, il, mid); break;
        case 8: hipLaunchKernelGGL(k_silu_mul<8>, grid, dim3(256), 0, st, big, part, L, I, il, mid); break;
        default: throw Error("silu_mul: unsupported partial count");
    }
    launched("silu_mul");
}

void add_bias(f16* y, int L, int N, const float* c, hipStream_t st) {
    const size_t n = (size_t)L * N;
    hipLaunchKernelGGL(k_add_bias, dim3((n + 255) / 256), dim3(256), 0, st, y, n, N, c);
    launched("add_bias");
}

namespace {
constexpr int kCopyBatch = 32;
struct CopyArgs {
    CopyDesc d[kCopyBatch];
};
// Descriptor blockIdx.y; the workgroups along x stride over its 16-byte chunks.
__global__ __launch_bounds__(256) void k_copy_batch(CopyArgs a) {
    const CopyDesc& d = a.d[blockIdx.y];
    const uint32_t per_row = (uint32_t)(d.row_bytes / 16);
    const uint64_t total = d.rows * per_row;
    for (uint64_t c = (uint64_t)blockIdx.x * 256 + threadIdx.x; c < total; c += (uint64_t)gridDim.x * 256) {
        const uint64_t r = c / per_row, o = (c % per_row) * 16;
        *reinterpret_cast<uint4*>(d.dst + r * d.dst_pitch + o) = *reinterpret_cast<const uint4*>(d.src + r * d.src_pitch + o);
    }
}
}  // namespace

void copy_batch(const CopyDesc* d, size_t n, hipStream_t st) {
    for (size_t i0 = 0; i0 < n; i0 += kCopyBatch) {
        const size_t m = std::min<size_t>(kCopyBatch, n - i0);
        CopyArgs a{};
        uint64_t most = 0;
        for (size_t i = 0; i < m; i++) {
            const CopyDesc& c = d[i0 + i];
            SD_CHECK(((uintptr_t)c.src | (uintptr_t)c.dst | c.row_bytes | c.src_pitch | c.dst_pitch) % 16 == 0,
                     "copy_batch: addresses, pitches and row sizes must be multiples of 16 bytes");
            a.d[i] = c;
            most = std::max(most, c.rows * c.row_bytes / 16);
        }
        if (most == 0) continue;
        const unsigned gx = (unsigned)std::min<uint64_t>((most + 255) / 256, 512);
        hipLaunchKernelGGL(k_copy_batch, dim3(gx, (unsigned)m), dim3(256), 0, st, a);
        launched("copy_batch");
    }
}

void set_u32x8(uint32_t* p, const uint32_t v[8], hipStream_t st) {
    U32x8 a;
    for (int i = 0; i < 8; i++) a.v[i] = v[i];
    hipLaunchKernelGGL(k_set_u32x8, dim3(1), dim3(64), 0, st, p, a);
    launched("set_u32x8");
}

void fill_u32(uint32_t* p, size_t n, uint32_t v, hipStream_t st) {
    if (n == 0) return;
    hipLaunchKernelGGL(k_fill_u32, dim3((n + 255) / 256), dim3(256), 0, st, p, n, v);
    launched("fill");
}

}  // namespace sd
