// Device-side helpers shared by the quantized GEMM and GEMV kernels: raw buffer loads (with their
// zero-filling range check), explicit vector-memory waits and barriers, and the int4 nibble dequant.
#pragma once

#include "common.h"

namespace sd {
namespace {

// The 8 nibbles of a weight word in the engine nibble order (see k_repack_w4) as 4 f16 pairs q - 8
// (exact) for k = (0,1), (2,3), (4,5), (6,7): the nibble at bits 4p lands in the f16 mantissa as
// 1024 + q for p = 0, 2 (and 4, 6 in the high half), as 1024 + 16 q for the others, so two masks per
// 8-bit shift give all four pairs.
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

// Raw buffer access (MUBUF): a 128-bit resource of base address and byte size, per-lane 32-bit
// offsets (VGPR) plus a uniform one (SGPR); an offset at or past the size reads zeros and touches no
// memory.  The host pass of hipcc does not see the builtins.
#if defined(__HIP_DEVICE_COMPILE__)
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
// 16 bytes per lane straight into LDS at lds + 16 lane (lds wave-uniform).
__device__ __forceinline__ void buf_lds16(Rsrc r, uint32_t voff, uint32_t soff, void* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ u32x4 buf_b128(Rsrc r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ uint32_t buf_b16(Rsrc r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}
__device__ __forceinline__ u32x3 buf_b96(Rsrc r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x3, __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, 0));
}
__device__ __forceinline__ u32x2 buf_b64(Rsrc r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}
__device__ __forceinline__ uint32_t buf_b32(Rsrc r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
// A 32-bit store; an offset at or past the resource's size writes nothing.
__device__ __forceinline__ void buf_st32(Rsrc r, uint32_t voff, uint32_t soff, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, voff, soff, 0);
}
#else
struct Rsrc {};
__device__ inline Rsrc make_rsrc(const void*, uint32_t) { return {}; }
__device__ inline void buf_lds16(Rsrc, uint32_t, uint32_t, void*) {}
__device__ inline u32x4 buf_b128(Rsrc, uint32_t, uint32_t) { return u32x4{}; }
__device__ inline uint32_t buf_b16(Rsrc, uint32_t, uint32_t) { return 0; }
__device__ inline u32x3 buf_b96(Rsrc, uint32_t, uint32_t) { return u32x3{}; }
__device__ inline u32x2 buf_b64(Rsrc, uint32_t, uint32_t) { return u32x2{}; }
__device__ inline uint32_t buf_b32(Rsrc, uint32_t, uint32_t) { return 0; }
__device__ inline void buf_st32(Rsrc, uint32_t, uint32_t, uint32_t) {}
#endif

// A per-lane buffer offset that is out of range for every buffer here: the load returns zeros and
// touches no memory.
constexpr uint32_t OOB = 0x80000000u;

// s_waitcnt immediate for vmcnt(v) with the lgkm and exp counters left unconstrained.
constexpr int vmcnt_imm(int v) { return 0x0F70 | (v & 15) | ((v >> 4) << 14); }

// s_waitcnt with a vmcnt that counts this thread's loads in issue order: scheduling barriers on
// both sides keep the compiler from moving loads across it, which would change what it counts.
template <int IMM>
__device__ __forceinline__ void wait_loads() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(IMM);
    __builtin_amdgcn_sched_barrier(0);
}

// Workgroup barrier without the release fence of __syncthreads, whose wait for every outstanding
// vector-memory load would drain the loads issued for later steps.  The caller waits (vmcnt) for
// the loads the other waves need; the "memory" clobber keeps the compiler from moving LDS
// accesses across.
__device__ __forceinline__ void bar_noflush() { asm volatile("s_barrier" ::: "memory"); }

// Workgroup barrier after this wave's LDS accesses have completed (outstanding global stores are
// not waited for, unlike __syncthreads).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// SGPR_BATCH("s"(x), "s"(y), ...): x, y, ... are in SGPRs at this point.  The scalar loads that
// produce them (kernel arguments past the preloaded ones, lu fields, table entries) are then issued
// as one batch and waited for together, one memory round trip, where the compiler would sink each
// load to its first use, behind branches, and wait for each in turn (scalar loads return out of
// order, so every wait is for all of them).
#define SGPR_BATCH(...) asm volatile("" ::__VA_ARGS__)

// XCD-aware tile order of a (gx column blocks, gy row blocks, gz K splits) grid: the hardware gives
// workgroup b to XCD b % 8, and each XCD has its own L2.  With a K split (gz in {2, 4, 8}) XCD x
// takes split x % gz and a contiguous run of the column-block-major (column, row) tiles, so it reads
// only that split's K range of the activations and of the weights.  Otherwise XCD x takes a
// contiguous run of the tiles in column-block-major order (every row block of a column block
// together), so a column block's weights reach one L2 only.
__device__ __forceinline__ void xcd_tile(int b, int gx, int gy, int gz, int& bx, int& by, int& bz) {
    const int G = gx * gy * gz, q8 = G >> 3;
    if (gz > 1 && 8 % gz == 0 && (G & 7) == 0) {
        const int x = b & 7, t = (x / gz) * q8 + (b >> 3);
        bz = x % gz;
        bx = t / gy;
        by = t % gy;
        return;
    }
    const int tile = b < 8 * q8 ? (b & 7) * q8 + (b >> 3) : b;
    const int gyz = gy * gz;
    bx = tile / gyz;
    by = (tile % gyz) % gy;
    bz = (tile % gyz) / gy;
}

// silu(g) * u = g / (1 + e^-g) * u on the hardware exp2 (v_exp_f32) and reciprocal (v_rcp_f32), each
// within about 1 ulp in f32, where libm's expf and an IEEE divide take ~25 VALU instructions; the
// result is rounded to f16 by the caller, as the reference stores mid (src/kernels.rs:123-135).
// The limits hold: e^-g overflows to inf for g -> -inf and the reciprocal gives 0.
__device__ __forceinline__ float silu_mul(float g, float u) {
#if defined(__HIP_DEVICE_COMPILE__)
    const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
    return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
#else
    return g * u;
#endif
}

// silu(x) = x / (1 + e^-x) the same way, kept in f32 (the conv output of the chunked delta rule;
// the reference's WGSL exp is no more exact than v_exp_f32).
__device__ __forceinline__ float silu(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
#else
    return x;
#endif
}

__device__ __forceinline__ f16x8 cat4(f16x2 a, f16x2 b, f16x2 c, f16x2 d) {
    return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

}  // namespace
}  // namespace sd
