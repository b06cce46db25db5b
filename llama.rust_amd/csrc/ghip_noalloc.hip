// ghip_noalloc.hip -- ghip_mul_mat_noalloc: GGML_OP_MUL_MAT without any
// allocation, on a fixed scratch array that lives in this library's own code
// object on every GPU it runs on.
//
// The array is a file-scope __device__ variable.  Its name in host code is
// only a host-side stand-in: the device address comes from
// hipGetSymbolAddress, looked up once per device at ghip_init (device
// current) and kept per device; kernels, copies and fills use that address.
#include <hip/hip_runtime.h>

#include <mutex>

#include "ghip_internal.h"

namespace {

// Decode GEMVs need at most a few MB (Q8 activation rows); the Q4_K prefill
// GEMM needs its Q8_K rows plus the GEMM layout (about 9.4 MB at 2048 tokens
// x 4096) and split-K partials for small grids.  The Q6_K prefill GEMM, which
// repacks its weights into the workspace per call, does not fit for large
// matrices and is refused.
constexpr size_t kScratchBytes = (size_t)32 << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
void *g_ptr[kMaxDevices];  // device address of `scratch` per device, once looked up

}  // namespace

ghip_status ghip_noalloc_setup(int device, const char **why) {
    if (device < 0 || device >= kMaxDevices) {
        *why = "device index out of range for the scratch table";
        return GHIP_STATUS_BACKEND_ERROR;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_ptr[device]) return GHIP_STATUS_SUCCESS;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        *why = "hipGetSymbolAddress(scratch) failed";
        return GHIP_STATUS_BACKEND_ERROR;
    }
    g_ptr[device] = p;
    return GHIP_STATUS_SUCCESS;
}

extern "C" ghip_status ghip_mul_mat_noalloc(ghip_context *ctx, const ghip_tensor *src0, const ghip_tensor *src1,
                                            const ghip_tensor *dst, void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    const int dev = ghip_context_device(ctx);
    void *p = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        if (dev >= 0 && dev < kMaxDevices) p = g_ptr[dev];
    }
    if (!p) return ghip_context_fail(ctx, GHIP_STATUS_BACKEND_ERROR, "mul_mat_noalloc: scratch not set up on this device");
    return ghip_mul_mat_fixed_scratch(ctx, src0, src1, dst, p, kScratchBytes, stream);
}
