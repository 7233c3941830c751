// The pointer head (src/head.rs:55-77) on the device, in f64 as the reference computes it on the
// host: LayerNorm (eps 1e-5) of each hidden row, the q projection of the answer row and the k
// projection of each option row, logits k.q * dim^-0.5 / max(T, 1e-6), softmax.  Also the optional
// unrotate of a rotated torso (src/engine.rs:652-660, 714-727), applied to the rows first.
#include "common.h"

namespace sd {
namespace {

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Sum over the 256 threads of the workgroup (every thread gets the result).
__device__ double block_sum_f64(double v, double* red) {
    v = wave_sum_f64(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// Row r: LayerNorm in f64 into LDS, then 16 outputs [16 y, 16 y + 16) of the q (answer row) or k
// projection.  Wave w takes columns [w d/4, (w + 1) d/4) of all 16 outputs, and the 4 partial dot
// products meet in LDS.  Every global load is unconditional (indices clamped, values masked after
// they arrive): a load under a branch would make the wave wait for it before issuing the next.
__global__ __launch_bounds__(256) void k_head_rows(const float* __restrict__ hid, int d, HeadW w,
                                                   const uint8_t* __restrict__ is_answer, double* __restrict__ proj) {
    extern __shared__ double xn[];  // d values
    __shared__ double red[4];
    __shared__ double part[4][16];
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* x = hid + (size_t)r * d;
#pragma unroll 4
    for (int j = 4 * tid; j < d; j += 1024) {
        const float4 v = *reinterpret_cast<const float4*>(x + j);
        xn[j] = (double)v.x, xn[j + 1] = (double)v.y, xn[j + 2] = (double)v.z, xn[j + 3] = (double)v.w;
    }
    __syncthreads();
    double s = 0.0;
    for (int j = tid; j < d; j += 256) s += xn[j];
    const double mean = block_sum_f64(s, red) / (double)d;
    double v = 0.0;
    for (int j = tid; j < d; j += 256) {
        const double t = xn[j] - mean;
        v += t * t;
    }
    const double rs = 1.0 / sqrt(block_sum_f64(v, red) / (double)d + 1e-5);
    for (int j = tid; j < d; j += 256) xn[j] = (xn[j] - mean) * rs * (double)w.nw[j] + (double)w.nb[j];
    __syncthreads();
    const bool ans = is_answer[r] != 0;
    const float* W = ans ? w.qw : w.kw;
    const float* B = ans ? w.qb : w.kb;
    const int ob = blockIdx.y * 16;
    const int no = min(16, w.dim - ob);
    const int span = d / 4;
    double acc[16];
#pragma unroll
    for (int u = 0; u < 16; u++) acc[u] = 0.0;
    for (int j0 = wave * span + 4 * lane; j0 < (wave + 1) * span; j0 += 256) {
        float4 wv[16];
#pragma unroll
        for (int u = 0; u < 16; u++) wv[u] = *reinterpret_cast<const float4*>(W + (size_t)min(ob + u, w.dim - 1) * d + j0);
        const double x0 = xn[j0], x1 = xn[j0 + 1], x2 = xn[j0 + 2], x3 = xn[j0 + 3];
#pragma unroll
        for (int u = 0; u < 16; u++)
            acc[u] += (double)wv[u].x * x0 + (double)wv[u].y * x1 + (double)wv[u].z * x2 + (double)wv[u].w * x3;
    }
#pragma unroll
    for (int u = 0; u < 16; u++) {
        const double a = wave_sum_f64(acc[u]);
        if (lane == 0) part[wave][u] = a;
    }
    __syncthreads();
    if (tid < no) proj[(size_t)r * w.dim + ob + tid] = (double)B[ob + tid] + ((part[0][tid] + part[1][tid]) + (part[2][tid] + part[3][tid]));
}

// Question q (one wave): rows [first, first + n) are its options, row first + n its answer.  The
// loads are unconditional (option rows past n read row first + n - 1, their sums unused).
__global__ __launch_bounds__(64) void k_head_probs(const double* __restrict__ proj, int dim,
                                                    const uint32_t* __restrict__ qtab, const double* __restrict__ scale,
                                                    const uint32_t* __restrict__ ooff, double* __restrict__ probs) {
    const int q = blockIdx.x, lane = threadIdx.x;
    const int first = (int)(qtab[q] & 0xFFFFu), n = (int)(qtab[q] >> 16);
    const double* qa = proj + (size_t)(first + n) * dim;
    double* out = probs + ooff[q];
    // logits: each option's k . q as a 64-lane dot product, 8 options at a time
    double mx = -INFINITY;
    for (int i0 = 0; i0 < n; i0 += 8) {
        double sv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) sv[u] = 0.0;
#pragma unroll 4
        for (int o = lane; o < dim; o += 64) {
            const double a = qa[o];
#pragma unroll
            for (int u = 0; u < 8; u++) sv[u] += proj[(size_t)(first + min(i0 + u, n - 1)) * dim + o] * a;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (i0 + u >= n) break;
            const double l = wave_sum_f64(sv[u]) * scale[q];
            if (lane == 0) out[i0 + u] = l;
            mx = fmax(mx, l);
        }
    }
    __syncthreads();  // out[] written by lane 0 is read by every lane below
    double z = 0.0;
    for (int i = lane; i < n; i += 64) {
        const double e = exp(out[i] - mx);
        out[i] = e;
        z += e;
    }
    z = wave_sum_f64(z);
    for (int i = lane; i < n; i += 64) out[i] /= z;
}

// In-place fast Walsh-Hadamard transform of each row (Sylvester order, unnormalised, f32 butterflies
// as on the host), then x[j] = f32(x[j] * unrotate[j]) in f64.
__global__ __launch_bounds__(256) void k_unrotate(float* __restrict__ rows, int d, const double* __restrict__ unrot) {
    extern __shared__ float xs[];
    float* x = rows + (size_t)blockIdx.x * d;
    for (int j = threadIdx.x; j < d; j += 256) xs[j] = x[j];
    __syncthreads();
    for (int h = 1; h < d; h *= 2) {
        for (int p = threadIdx.x; p < d / 2; p += 256) {
            const int j = (p / h) * 2 * h + (p % h);
            const float a = xs[j], b = xs[j + h];
            xs[j] = a + b;
            xs[j + h] = a - b;
        }
        __syncthreads();
    }
    for (int j = threadIdx.x; j < d; j += 256) x[j] = (float)((double)xs[j] * unrot[j]);
}

}  // namespace

void head_rows(const float* hidden, int n_rows, int d, const HeadW& w, const uint8_t* is_answer, double* proj,
               hipStream_t st) {
    SD_CHECK(d % 256 == 0 && w.dim > 0, "head: hidden size must be a multiple of 256");
    SD_CHECK(d % 16 == 0, "head: hidden size must be a multiple of 16");
    hipLaunchKernelGGL(k_head_rows, dim3(n_rows, (w.dim + 15) / 16), dim3(256), (size_t)d * 8, st, hidden, d, w,
                       is_answer, proj);
    launched("head_rows");
}

void head_probs(const double* proj, int dim, const uint32_t* qtab, const double* scale, const uint32_t* ooff, int nq,
                double* probs, hipStream_t st) {
    hipLaunchKernelGGL(k_head_probs, dim3(nq), dim3(64), 0, st, proj, dim, qtab, scale, ooff, probs);
    launched("head_probs");
}

void unrotate_rows(float* rows, int n_rows, int d, const double* unrot, hipStream_t st) {
    SD_CHECK((d & (d - 1)) == 0, "unrotate: hidden size must be a power of two");
    hipLaunchKernelGGL(k_unrotate, dim3(n_rows), dim3(256), (size_t)d * 4, st, rows, d, unrot);
    launched("unrotate");
}

}  // namespace sd
