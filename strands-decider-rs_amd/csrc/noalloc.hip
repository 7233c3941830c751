// sd_op_matmul_noalloc: sd_op_matmul for callers that cannot allocate device memory (code under HIP
// graph capture, tight serving loops).  The split-K partial slots that sd_op_matmul keeps in a
// workspace it grows with hipMalloc live here in a fixed device array instead.
#include <mutex>

#include "../../include/sdhip.h"
#include "common.h"

namespace {

// The split-K partial slots ([ks][M][N] f32) of every call on a device: 16 MiB, fixed.  Each GPU the
// library runs on holds its own copy of this array until the process ends.  Host code must not use
// this name as a device address; it uses the address hipGetSymbolAddress returns for the device.
constexpr size_t SCRATCH_FLOATS = size_t(4) << 20;
static __device__ __align__(256) float scratch[SCRATCH_FLOATS];

// The device address of `scratch` on each device, looked up once per device with that device
// current, on the first call that needs it (so a caller about to capture a graph makes one call
// first: the lookup is then not part of the capture).
std::mutex scratch_mu;
float* scratch_dev[64] = {};

float* scratch_ptr() {
    int dev = 0;
    SD_HIP(hipGetDevice(&dev));
    SD_CHECK(dev >= 0 && dev < 64, "sd_op_matmul_noalloc: device index out of range");
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_dev[dev]) {
        void* p = nullptr;
        SD_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        SD_CHECK(p != nullptr, "sd_op_matmul_noalloc: no device address for the scratch array");
        scratch_dev[dev] = static_cast<float*>(p);
    }
    return scratch_dev[dev];
}

void put_err(char* err, size_t errlen, const char* msg) {
    if (!err || errlen == 0) return;
    size_t i = 0;
    for (; msg[i] && i + 1 < errlen; i++) err[i] = msg[i];
    err[i] = '\0';
}

}  // namespace

extern "C" int sd_op_matmul_noalloc(const void* A, const void* Wq, const void* Sc, void* Y, int M, int N, int K, int exact,
                                    void* stream, char* err, size_t errlen) {
    try {
        if (!A || !Wq || !Sc || !Y) throw sd::Error("sd_op_matmul_noalloc: null argument");
        if (M < 1 || N < 1 || K < 128 || K % 128)
            throw sd::Error("sd_op_matmul_noalloc: need M, N >= 1 and K a multiple of 128");
        const bool tiled = sd::w4_tileable(N, K);
        const hipStream_t st = static_cast<hipStream_t>(stream);
        const auto* a = static_cast<const sd::f16*>(A);
        const auto* wq = static_cast<const uint32_t*>(Wq);
        const auto* sc = static_cast<const sd::f16*>(Sc);
        if (exact) {
            // the GEMV rows: no scratch (the weights as sd_op_repack_w4 left them)
            sd::gemv(a, wq, sc, nullptr, Y, 0, M, N, K, 4, 32, false, tiled, sd::gemv_plan(M, N, K, tiled, 0, 0), st);
        } else {
            if (!tiled)
                throw sd::Error("sd_op_matmul_noalloc: the f16-dequant kernels need N a multiple of 32 here "
                                "(other shapes are rewritten into a workspace: use sd_op_matmul)");
            // the plan sd_op_matmul takes for this shape (the same kernels, splits and results); when
            // its split-K slots do not fit the array, the same kernel with the largest split that
            // fits (down to none), whose slots add in another order
            sd::GemmPlan p = sd::gemm_w4_plan(M, N, K, false, true, size_t(64) << 20);
            if ((size_t)p.ks * M * N > SCRATCH_FLOATS) p = sd::gemm_w4_plan(M, N, K, false, true, SCRATCH_FLOATS);
            if (p.ks == 1) {
                sd::gemm_w4(a, wq, sc, static_cast<sd::f16*>(Y), nullptr, M, N, K, false, 1, st, p.cfg, true);
            } else {
                SD_CHECK((size_t)p.ks * M * N <= SCRATCH_FLOATS, "sd_op_matmul_noalloc: the split does not fit the scratch array");
                float* part = scratch_ptr();
                sd::gemm_w4(a, wq, sc, nullptr, part, M, N, K, false, p.ks, st, p.cfg, true);
                sd::reduce_partials(part, p.ks, (size_t)M * N, static_cast<sd::f16*>(Y), st);
            }
        }
        if (err && errlen) err[0] = '\0';
        return 0;
    } catch (const std::exception& e) {
        put_err(err, errlen, e.what());
    } catch (...) {
        put_err(err, errlen, "unknown error");
    }
    return 1;
}
