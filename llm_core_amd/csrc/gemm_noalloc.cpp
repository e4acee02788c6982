// gemm_noalloc.cpp — axf_hip_gemm_q4k_q8_noalloc: the Q4_K x Q8_0 small-M GEMM
// of axf_hip_gemm_q4k_q8 for callers that cannot allocate device memory.
//
// The matrix-core paths need a scratch buffer: the LDS-ring kernel's re-laid
// Q8_0 activations (k_gemm_prep / k_gemm_prep16 write every byte of it, token
// padding included), or the register-weights kernel's split-K partial sums
// (every element written before it is summed); nothing needs clearing.  axf_hip_gemm_q4k_q8
// takes that buffer from the context, growing it with hipMalloc.  Here it
// is `scratch`, a file-scope device array of kNoAllocScratchBytes: each GPU
// the library runs on holds its own copy until the process ends.  Its device
// address is looked up once per device (hipGetSymbolAddress, with that device
// current) and kept in g_scratch_ptr; host code passes only that address to
// the kernels, never the array's name (a host-side stand-in).
//
// Calls on one GPU share the array: two calls whose kernels overlap (on
// different streams or contexts of one device) race on it.
#include <mutex>

#include "capi_internal.hpp"

constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;  // 8 MiB per device

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's `scratch`, looked up on the first call.
int scratch_address(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices)
        return axf::fail(AXF_ERR_UNSUPPORTED, "axf_hip_gemm_q4k_q8_noalloc: device index above 63");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != device) e = hipSetDevice(device);
        void* p = nullptr;
        if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur >= 0 && cur != device) (void)hipSetDevice(cur);
        if (e != hipSuccess) return axf::hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) return axf::fail(AXF_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return AXF_OK;
}

}  // namespace

extern "C" int axf_hip_gemm_q4k_q8_noalloc(axf_ctx* ctx, float* Y, const void* W,
                                           const void* XQ8, int rows, int T, int cols,
                                           size_t row_bytes) {
    using namespace axf;
    const char* fn = "axf_hip_gemm_q4k_q8_noalloc";
    if (!ctx) return fail(AXF_ERR_INVALID_ARG, std::string(fn) + ": null context");
    if (T < 0) return fail(AXF_ERR_INVALID_ARG, std::string(fn) + ": negative T");
    int rc = check_gemv(fn, AXF_TYPE_Q4_K, W, XQ8, Y, rows, cols, row_bytes, false);
    if (rc) return rc;
    if (rows == 0 || cols == 0 || T == 0) return AXF_OK;
    // the automatic choice, or the LDS-ring kernel where that needs less scratch
    GemmPath path = GemmPath::Auto;
    size_t need = gemm_scratch_bytes(AXF_TYPE_Q4_K, path, T, cols / QK_K, rows);
    if (need > kNoAllocScratchBytes) {
        path = GemmPath::Mfma;
        need = gemm_scratch_bytes(AXF_TYPE_Q4_K, path, T, cols / QK_K, rows);
    }
    if (need > kNoAllocScratchBytes)
        return fail(AXF_ERR_INVALID_ARG,
                    std::string(fn) + ": T = " + std::to_string(T) + " tokens at cols = " +
                        std::to_string(cols) + " need " + std::to_string(need) +
                        " bytes of scratch, above the fixed " +
                        std::to_string(kNoAllocScratchBytes) + " (use axf_hip_gemm_q4k_q8)");
    void* sp = nullptr;
    if (need) {
        rc = scratch_address(ctx->device, &sp);
        if (rc) return rc;
    }
    hipError_t e = launch_gemm_q4k_q8(Y, W, XQ8, rows, T, cols / QK_K, (long)row_bytes, path,
                                      sp, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, fn);
    return AXF_OK;
}
