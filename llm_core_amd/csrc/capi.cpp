// capi.cpp — C-ABI entry points of libaxf_hip.so (declared in include/axf_hip.h).
#include "capi_internal.hpp"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>

namespace axf {

static thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char* where) {
    return fail(AXF_ERR_HIP, std::string(where) + ": " + hipGetErrorString(e));
}

int ctx_scratch(axf_ctx* ctx, size_t bytes, void** p) {
    if (ctx->scratch_bytes < bytes) {
        if (ctx->scratch) (void)hipFree(ctx->scratch);
        ctx->scratch = nullptr;
        ctx->scratch_bytes = 0;
        size_t sz = bytes < (1u << 20) ? (1u << 20) : bytes;
        hipError_t e = hipMalloc(&ctx->scratch, sz);
        if (e != hipSuccess) return hip_fail(e, "hipMalloc(scratch)");
        ctx->scratch_bytes = sz;
    }
    *p = ctx->scratch;
    return AXF_OK;
}

}  // namespace axf

using namespace axf;

#define AXF_CHECK_CTX(ctx) \
    if (!(ctx)) return fail(AXF_ERR_INVALID_ARG, std::string(__func__) + ": null context")
#define AXF_REQUIRE(cond, msg) \
    if (!(cond)) return fail(AXF_ERR_INVALID_ARG, std::string(__func__) + ": " + (msg))
#define AXF_HIP(call)                                          \
    do {                                                       \
        hipError_t e_ = (call);                                \
        if (e_ != hipSuccess) return hip_fail(e_, __func__);   \
    } while (0)

static inline bool aligned(const void* p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

extern "C" {

const char* axf_hip_last_error(void) { return g_last_error.c_str(); }

int axf_hip_version(int* major, int* minor, int* patch) {
    if (major) *major = 0;
    if (minor) *minor = 1;
    if (patch) *patch = 0;
    return AXF_OK;
}

int axf_hip_device_count(int* count) {
    AXF_REQUIRE(count, "null count");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;
    *count = n;
    return AXF_OK;
}

int axf_hip_create(int device, axf_ctx** out) {
    AXF_REQUIRE(out, "null out");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        return fail(AXF_ERR_NO_DEVICE, "axf_hip_create: no HIP device");
    AXF_REQUIRE(device >= 0 && device < n, "device index out of range");
    AXF_HIP(hipSetDevice(device));
    auto* ctx = new axf_ctx();
    ctx->device = device;
    hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&ctx->ev0);
    if (e == hipSuccess) e = hipEventCreate(&ctx->ev1);
    if (e != hipSuccess) {
        delete ctx;
        return hip_fail(e, "axf_hip_create");
    }
    *out = ctx;
    return AXF_OK;
}

int axf_hip_destroy(axf_ctx* ctx) {
    if (!ctx) return AXF_OK;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    (void)hipEventDestroy(ctx->ev0);
    (void)hipEventDestroy(ctx->ev1);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return AXF_OK;
}

int axf_hip_device_name(axf_ctx* ctx, char* buf, int buflen) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(buf && buflen > 0, "null buffer");
    hipDeviceProp_t prop;
    AXF_HIP(hipGetDeviceProperties(&prop, ctx->device));
    std::snprintf(buf, (size_t)buflen, "%s (%s, %d CUs)", prop.name, prop.gcnArchName,
                  prop.multiProcessorCount);
    return AXF_OK;
}

int axf_hip_alloc(axf_ctx* ctx, size_t bytes, void** dptr) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(dptr, "null out pointer");
    *dptr = nullptr;
    if (bytes == 0) return AXF_OK;
    AXF_HIP(hipMalloc(dptr, bytes));
    return AXF_OK;
}

int axf_hip_free(axf_ctx* ctx, void* dptr) {
    AXF_CHECK_CTX(ctx);
    if (dptr) AXF_HIP(hipFree(dptr));
    return AXF_OK;
}

int axf_hip_memcpy_h2d(axf_ctx* ctx, void* dst, const void* src, size_t bytes) {
    AXF_CHECK_CTX(ctx);
    if (!bytes) return AXF_OK;
    AXF_REQUIRE(dst && src, "null pointer");
    AXF_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    AXF_HIP(hipStreamSynchronize(ctx->stream));
    return AXF_OK;
}

int axf_hip_memcpy_d2h(axf_ctx* ctx, void* dst, const void* src, size_t bytes) {
    AXF_CHECK_CTX(ctx);
    if (!bytes) return AXF_OK;
    AXF_REQUIRE(dst && src, "null pointer");
    AXF_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    AXF_HIP(hipStreamSynchronize(ctx->stream));
    return AXF_OK;
}

int axf_hip_memcpy_d2d(axf_ctx* ctx, void* dst, const void* src, size_t bytes) {
    AXF_CHECK_CTX(ctx);
    if (!bytes) return AXF_OK;
    AXF_REQUIRE(dst && src, "null pointer");
    AXF_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return AXF_OK;
}

int axf_hip_sync(axf_ctx* ctx) {
    AXF_CHECK_CTX(ctx);
    AXF_HIP(hipStreamSynchronize(ctx->stream));
    return AXF_OK;
}

// ---------------------------------------------------------------------------

int axf_hip_dequant_q4k(axf_ctx* ctx, float* y, const void* W, int64_t n_blocks) {
    AXF_CHECK_CTX(ctx);
    if (n_blocks == 0) return AXF_OK;
    AXF_REQUIRE(n_blocks > 0 && y && W, "bad arguments");
    AXF_REQUIRE(aligned(W, 16) && aligned(y, 16), "W and y must be 16-byte aligned");
    AXF_HIP(launch_dequant_q4k(y, W, (long)n_blocks, ctx->stream));
    return AXF_OK;
}

int axf_hip_dequant_q6k(axf_ctx* ctx, float* y, const void* W, int64_t n_blocks) {
    AXF_CHECK_CTX(ctx);
    if (n_blocks == 0) return AXF_OK;
    AXF_REQUIRE(n_blocks > 0 && y && W, "bad arguments");
    AXF_REQUIRE(aligned(W, 2) && aligned(y, 4), "W must be 2-byte and y 4-byte aligned");
    AXF_HIP(launch_dequant_q6k(y, W, (long)n_blocks, ctx->stream));
    return AXF_OK;
}

int axf_hip_quantize_q8_0(axf_ctx* ctx, void* xq8, const float* x, int n) {
    AXF_CHECK_CTX(ctx);
    if (n == 0) return AXF_OK;
    AXF_REQUIRE(n > 0 && n % 32 == 0, "n must be a positive multiple of 32");
    AXF_REQUIRE(xq8 && x && aligned(x, 16) && aligned(xq8, 4), "bad pointers/alignment");
    AXF_HIP(launch_quantize_q8_0(xq8, x, n, ctx->stream));
    return AXF_OK;
}

}  // extern "C"

int axf::check_gemv(const char* fn, int qtype, const void* W, const void* x, const float* y,
                    int rows, int cols, size_t row_bytes, bool f32x) {
    if (rows < 0 || cols < 0) return fail(AXF_ERR_INVALID_ARG, std::string(fn) + ": negative size");
    if (cols % QK_K != 0)
        return fail(AXF_ERR_INVALID_ARG, std::string(fn) + ": cols must be a multiple of 256");
    const int nb = cols / QK_K;
    if (nb > kMaxBlocksPerRow)
        return fail(AXF_ERR_UNSUPPORTED, std::string(fn) + ": cols > 32768 not supported");
    const size_t min_rb = (size_t)nb * (qtype == AXF_TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES);
    if (row_bytes < min_rb)
        return fail(AXF_ERR_INVALID_ARG, std::string(fn) + ": row_bytes smaller than one row");
    if (!W || !x || !y) return fail(AXF_ERR_INVALID_ARG, std::string(fn) + ": null pointer");
    if (qtype == AXF_TYPE_Q4_K) {
        if (!aligned(W, 16) || row_bytes % 16)
            return fail(AXF_ERR_INVALID_ARG,
                        std::string(fn) + ": Q4_K needs 16-byte aligned W and row_bytes");
    } else {
        if (!aligned(W, 4) || row_bytes % 2)
            return fail(AXF_ERR_INVALID_ARG,
                        std::string(fn) + ": Q6_K needs 4-byte aligned W and even row_bytes");
    }
    if (!aligned(y, 4)) return fail(AXF_ERR_INVALID_ARG, std::string(fn) + ": y misaligned");
    if (f32x) {
        if (!aligned(x, 16)) return fail(AXF_ERR_INVALID_ARG, std::string(fn) + ": x misaligned");
        const size_t lds = (size_t)cols * 4 * (qtype == AXF_TYPE_Q4_K ? 17 : 18) / 16;
        if (lds > 65536)
            return fail(AXF_ERR_UNSUPPORTED, std::string(fn) + ": cols too large for F32 path");
    } else if (!aligned(x, 4)) {
        return fail(AXF_ERR_INVALID_ARG, std::string(fn) + ": xq8 misaligned");
    }
    return AXF_OK;
}

extern "C" {

static int do_gemv(axf_ctx* ctx, const char* fn, GemvKind kind, int qtype, float* y,
                   const void* W, const void* x, int rows, int cols, size_t row_bytes,
                   int accumulate) {
    if (!ctx) return fail(AXF_ERR_INVALID_ARG, std::string(fn) + ": null context");
    const bool f32x = (kind == GemvKind::Q4K_F32 || kind == GemvKind::Q6K_F32);
    int rc = check_gemv(fn, qtype, W, x, y, rows, cols, row_bytes, f32x);
    if (rc) return rc;
    if (rows == 0 || cols == 0) return AXF_OK;
    hipError_t e = launch_gemv(kind, y, W, x, rows, cols / QK_K, (long)row_bytes,
                               accumulate ? 1 : 0, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, fn);
    return AXF_OK;
}

int axf_hip_gemv_q4k_f32(axf_ctx* ctx, float* y, const void* W, const float* x, int rows,
                         int cols, size_t row_bytes) {
    return do_gemv(ctx, __func__, GemvKind::Q4K_F32, AXF_TYPE_Q4_K, y, W, x, rows, cols,
                   row_bytes, 0);
}
int axf_hip_gemv_q6k_f32(axf_ctx* ctx, float* y, const void* W, const float* x, int rows,
                         int cols, size_t row_bytes) {
    return do_gemv(ctx, __func__, GemvKind::Q6K_F32, AXF_TYPE_Q6_K, y, W, x, rows, cols,
                   row_bytes, 0);
}
int axf_hip_gemv_q4k_q8(axf_ctx* ctx, float* y, const void* W, const void* xq8, int rows,
                        int cols, size_t row_bytes, int accumulate) {
    return do_gemv(ctx, __func__, GemvKind::Q4K_Q8, AXF_TYPE_Q4_K, y, W, xq8, rows, cols,
                   row_bytes, accumulate);
}
int axf_hip_gemv_q6k_q8(axf_ctx* ctx, float* y, const void* W, const void* xq8, int rows,
                        int cols, size_t row_bytes, int accumulate) {
    return do_gemv(ctx, __func__, GemvKind::Q6K_Q8, AXF_TYPE_Q6_K, y, W, xq8, rows, cols,
                   row_bytes, accumulate);
}

static int do_gemm(axf_ctx* ctx, const char* fn, int qtype, float* Y, const void* W,
                   const void* XQ8, int rows, int T, int cols, size_t row_bytes, int path) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(T >= 0, "negative T");
    AXF_REQUIRE(path >= 0 && path <= 3,
                "path must be 0 (auto), 1 (dot4), 2 (matrix cores) or 3 (matrix cores, streamed)");
    int rc = check_gemv(fn, qtype, W, XQ8, Y, rows, cols, row_bytes, false);
    if (rc) return rc;
    if (rows == 0 || cols == 0 || T == 0) return AXF_OK;
    const size_t sb = gemm_scratch_bytes(qtype, (GemmPath)path, T, cols / QK_K, rows);
    void* scratch = nullptr;
    if (sb) {
        rc = ctx_scratch(ctx, sb, &scratch);
        if (rc) return rc;
    }
    if (qtype == AXF_TYPE_Q6_K)
        AXF_HIP(launch_gemm_q6k_q8(Y, W, XQ8, rows, T, cols / QK_K, (long)row_bytes,
                                   (GemmPath)path, scratch, ctx->stream));
    else
        AXF_HIP(launch_gemm_q4k_q8(Y, W, XQ8, rows, T, cols / QK_K, (long)row_bytes,
                                   (GemmPath)path, scratch, ctx->stream));
    return AXF_OK;
}

int axf_hip_gemm_q4k_q8(axf_ctx* ctx, float* Y, const void* W, const void* XQ8, int rows, int T,
                        int cols, size_t row_bytes) {
    return do_gemm(ctx, __func__, AXF_TYPE_Q4_K, Y, W, XQ8, rows, T, cols, row_bytes, 0);
}

int axf_hip_gemm_q6k_q8(axf_ctx* ctx, float* Y, const void* W, const void* XQ8, int rows, int T,
                        int cols, size_t row_bytes) {
    return do_gemm(ctx, __func__, AXF_TYPE_Q6_K, Y, W, XQ8, rows, T, cols, row_bytes, 0);
}

int axf_hip_gemm_q6k_q8_path(axf_ctx* ctx, float* Y, const void* W, const void* XQ8, int rows,
                             int T, int cols, size_t row_bytes, int path) {
    return do_gemm(ctx, __func__, AXF_TYPE_Q6_K, Y, W, XQ8, rows, T, cols, row_bytes, path);
}

int axf_hip_gemm_q4k_q8_path(axf_ctx* ctx, float* Y, const void* W, const void* XQ8, int rows,
                             int T, int cols, size_t row_bytes, int path) {
    return do_gemm(ctx, __func__, AXF_TYPE_Q4_K, Y, W, XQ8, rows, T, cols, row_bytes, path);
}

int axf_hip_argmax_f32(axf_ctx* ctx, int* idx_dev, const float* x, int n) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(idx_dev && x && n > 0, "bad arguments");
    void* scratch = nullptr;
    const int parts = argmax_parts();
    int rc = ctx_scratch(ctx, (size_t)parts * 8, &scratch);
    if (rc) return rc;
    float* pv = static_cast<float*>(scratch);
    int* pi = reinterpret_cast<int*>(pv + parts);
    AXF_HIP(launch_argmax(idx_dev, pv, pi, x, n, nullptr, nullptr, nullptr, ctx->stream));
    return AXF_OK;
}

int axf_hip_sample(axf_ctx* ctx, float* logits_dev, int n_vocab, const axf_sampling* s,
                   const int32_t* hist, int n_hist, float r, int32_t* token) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(logits_dev && s && token && n_vocab > 0 && n_hist >= 0 && (n_hist == 0 || hist),
                "bad arguments");
    const int n_cand = sample_candidates(n_vocab, sample_k(*s, n_vocab));
    if (n_cand == 0)
        return fail(AXF_ERR_UNSUPPORTED, "axf_hip_sample: top_k too large for the device sampler");
    // scratch: candidates | history | history count | token
    const size_t hist_off = (size_t)n_cand * 8;
    const size_t bytes = hist_off + (size_t)(n_hist + 2) * 4;
    void* scratch = nullptr;
    int rc = ctx_scratch(ctx, bytes, &scratch);
    if (rc) return rc;
    auto* cand = static_cast<uint64_t*>(scratch);
    int* d_hist = reinterpret_cast<int*>(static_cast<uint8_t*>(scratch) + hist_off);
    int* d_hist_n = d_hist + n_hist;
    int* d_tok = d_hist_n + 1;
    if (s->rep_penalty != 1.0f && n_hist > 0) {
        AXF_HIP(hipMemcpyAsync(d_hist, hist, (size_t)n_hist * 4, hipMemcpyHostToDevice,
                               ctx->stream));
        AXF_HIP(hipMemcpyAsync(d_hist_n, &n_hist, 4, hipMemcpyHostToDevice, ctx->stream));
        AXF_HIP(launch_rep_penalty(logits_dev, d_hist, d_hist_n, s->rep_penalty_last_n,
                                   s->rep_penalty, n_vocab, ctx->stream));
    }
    AXF_HIP(launch_sample(d_tok, cand, logits_dev, n_vocab, s->temperature, s->top_k, s->top_p,
                          nullptr, r, nullptr, nullptr, nullptr, nullptr, nullptr, ctx->stream));
    AXF_HIP(hipMemcpyAsync(token, d_tok, 4, hipMemcpyDeviceToHost, ctx->stream));
    AXF_HIP(hipStreamSynchronize(ctx->stream));
    return AXF_OK;
}

int axf_hip_rmsnorm(axf_ctx* ctx, float* y, void* yq8, const float* x, const float* w, int n,
                    float eps) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(n > 0 && n % 32 == 0, "n must be a positive multiple of 32");
    AXF_REQUIRE(x && w && (y || yq8), "bad pointers");
    AXF_REQUIRE(aligned(x, 16) && aligned(w, 16) && (!y || aligned(y, 16)) &&
                    (!yq8 || aligned(yq8, 4)),
                "misaligned pointer");
    AXF_HIP(launch_rmsnorm(y, yq8, x, w, n, eps, ctx->stream));
    return AXF_OK;
}

int axf_hip_rope(axf_ctx* ctx, float* dst, const float* src, int pos, int n_heads, int head_dim,
                 const float* cos_t, const float* sin_t) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(dst && src && cos_t && sin_t, "null pointer");
    AXF_REQUIRE(pos >= 0 && n_heads > 0 && head_dim > 0 && head_dim % 2 == 0, "bad shape");
    AXF_HIP(launch_rope(dst, src, nullptr, pos, n_heads, head_dim, cos_t, sin_t, ctx->stream));
    return AXF_OK;
}

int axf_hip_attn_decode(axf_ctx* ctx, float* out, void* outq8, const float* q,
                        const float* kcache, const float* vcache, int seq, int n_heads,
                        int n_kv_heads, int head_dim) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(out && q && kcache && vcache, "null pointer");
    AXF_REQUIRE(seq > 0 && n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                "bad shape");
    AXF_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
                "head_dim must be 64, 128 or 256");
    AXF_REQUIRE(aligned(q, 4) && aligned(kcache, 16) && aligned(vcache, 16) && aligned(out, 4) &&
                    aligned(outq8, 4),
                "misaligned pointer");
    AXF_REQUIRE(n_heads / n_kv_heads <= 8, "more than 8 query heads per kv head");
    const int nsplit = attn_nsplit(seq);
    AXF_REQUIRE(nsplit <= 512, "seq above 32768");
    void* scratch = nullptr;
    int rc = ctx_scratch(ctx, (size_t)n_heads * nsplit * (head_dim + 2) * 4, &scratch);
    if (rc) return rc;
    AttnArgs a{};
    a.q = q;
    a.kcache = const_cast<float*>(kcache);
    a.vcache = const_cast<float*>(vcache);
    a.pos = seq - 1;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.nsplit = nsplit;
    a.store_kv = 0;
    a.part = static_cast<float*>(scratch);
    a.out = out;
    a.outq8 = static_cast<uint8_t*>(outq8);
    AXF_HIP(launch_attention_fused(a, head_dim, ctx->stream));
    return AXF_OK;
}

int axf_hip_attn_prefill(axf_ctx* ctx, float* out, void* outq8, const float* q, int q_ld,
                         const float* bq, const float* kcache, const float* vcache, int pos0,
                         int T, int n_heads, int n_kv_heads, int head_dim, const float* cos_t,
                         const float* sin_t, int path) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(out && q && kcache && vcache && cos_t && sin_t, "null pointer");
    AXF_REQUIRE(T > 0 && pos0 >= 0 && n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                "bad shape");
    AXF_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
                "head_dim must be 64, 128 or 256");
    AXF_REQUIRE(n_heads / n_kv_heads <= 8, "more than 8 query heads per kv head");
    AXF_REQUIRE(q_ld >= n_heads * head_dim, "q_ld below one row");
    AXF_REQUIRE(path == 0 || path == 1, "path must be 0 or 1");
    AXF_REQUIRE(aligned(q, 4) && aligned(kcache, 16) && aligned(vcache, 16) && aligned(out, 4) &&
                    aligned(outq8, 4),
                "misaligned pointer");
    const int nsplit = attn_nsplit(pos0 + T);
    AXF_REQUIRE(nsplit <= 512, "positions above 32768");
    AttnArgs a{};
    a.q = q;
    a.bq = bq;
    a.cos_t = cos_t;
    a.sin_t = sin_t;
    a.kcache = const_cast<float*>(kcache);
    a.vcache = const_cast<float*>(vcache);
    a.pos = pos0;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.nsplit = nsplit;
    a.store_kv = 0;
    a.out = out;
    a.outq8 = static_cast<uint8_t*>(outq8);
    a.n_tok = T;
    a.q_ld = q_ld;
    a.out_ld = n_heads * head_dim;
    if (path == 1) {
        void* scratch = nullptr;
        int rc = ctx_scratch(ctx, (size_t)T * n_heads * nsplit * (head_dim + 2) * 4, &scratch);
        if (rc) return rc;
        a.part = static_cast<float*>(scratch);
        AXF_HIP(launch_attention_fused(a, head_dim, ctx->stream));
    } else {
        AXF_HIP(launch_attention_prefill(a, head_dim, ctx->stream));
    }
    return AXF_OK;
}

int axf_hip_swiglu(axf_ctx* ctx, float* out, void* outq8, const float* gate, const float* up,
                   int n) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(n > 0 && n % 32 == 0, "n must be a positive multiple of 32");
    AXF_REQUIRE(gate && up && (out || outq8), "null pointer");
    AXF_REQUIRE(aligned(gate, 16) && aligned(up, 16) && (!out || aligned(out, 16)),
                "misaligned pointer");
    AXF_HIP(launch_swiglu(out, outq8, gate, up, n, ctx->stream));
    return AXF_OK;
}

int axf_hip_add(axf_ctx* ctx, float* y, const float* a, const float* b, int n) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(y && a && b && n >= 0, "bad arguments");
    if (n == 0) return AXF_OK;
    AXF_HIP(launch_add(y, a, b, n, ctx->stream));
    return AXF_OK;
}

int axf_hip_embed(axf_ctx* ctx, float* out, int qtype, const void* W, int token, int rows,
                  int cols) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(out && W && cols > 0, "bad arguments");
    AXF_REQUIRE(token >= 0 && token < rows, "token out of range");
    if (qtype == AXF_TYPE_Q8_0 || qtype == AXF_TYPE_Q5_0 || qtype == AXF_TYPE_F16) {
        AXF_REQUIRE(cols % 32 == 0, "cols must be a multiple of 32");
        AXF_REQUIRE(aligned(W, 2), "W misaligned");
        AXF_HIP(launch_embed_misc(qtype, out, W, nullptr, token, 1, cols,
                                  (long)axf_row_bytes(qtype, cols), ctx->stream));
        return AXF_OK;
    }
    AXF_REQUIRE(cols % QK_K == 0, "cols must be a multiple of 256");
    AXF_REQUIRE(qtype == AXF_TYPE_Q4_K || qtype == AXF_TYPE_Q6_K,
                "qtype must be Q4_K, Q6_K, Q8_0, Q5_0 or F16");
    AXF_REQUIRE(qtype == AXF_TYPE_Q6_K ? aligned(W, 2) : aligned(W, 16), "W misaligned");
    const int nb = cols / QK_K;
    AXF_HIP(launch_embed(qtype, out, W, nullptr, token, nb,
                         (long)axf_row_bytes(qtype, cols), ctx->stream));
    return AXF_OK;
}

// The other weight types: rows of cols/32 blocks (2-byte aligned) or halfs.
static int check_misc(const char* fn, int qtype, const void* W, const void* x, const float* y,
                      int rows, int cols, size_t row_bytes, bool x16) {
    const std::string f(fn);
    if (!W || !x || !y) return fail(AXF_ERR_INVALID_ARG, f + ": null pointer");
    if (rows < 0 || cols < 0) return fail(AXF_ERR_INVALID_ARG, f + ": negative size");
    if (qtype == AXF_TYPE_F16) {
        if (cols % 8) return fail(AXF_ERR_INVALID_ARG, f + ": cols must be a multiple of 8");
        if (!aligned(W, 16)) return fail(AXF_ERR_INVALID_ARG, f + ": W must be 16-byte aligned");
    } else {
        if (cols % 32) return fail(AXF_ERR_INVALID_ARG, f + ": cols must be a multiple of 32");
        if (row_bytes < axf_row_bytes(qtype, cols) || row_bytes % 2)
            return fail(AXF_ERR_INVALID_ARG, f + ": row_bytes smaller than one row or odd");
        if (!aligned(W, 2)) return fail(AXF_ERR_INVALID_ARG, f + ": W must be 2-byte aligned");
    }
    if (!aligned(x, x16 ? 16 : 4) || !aligned(y, 4))
        return fail(AXF_ERR_INVALID_ARG, f + ": x or y misaligned");
    return AXF_OK;
}

int axf_hip_gemv_q8_0w_q8(axf_ctx* ctx, float* y, const void* W, const void* xq8, int rows,
                          int cols, size_t row_bytes, int accumulate) {
    AXF_CHECK_CTX(ctx);
    int rc = check_misc(__func__, AXF_TYPE_Q8_0, W, xq8, y, rows, cols, row_bytes, false);
    if (rc) return rc;
    if (!rows || !cols) return AXF_OK;
    AXF_HIP(launch_gemv_q8w_q8(y, W, xq8, rows, cols / 32, (long)row_bytes, accumulate,
                               ctx->stream));
    return AXF_OK;
}

int axf_hip_gemv_q8_0w_f32(axf_ctx* ctx, float* y, const void* W, const float* x, int rows,
                           int cols, size_t row_bytes) {
    AXF_CHECK_CTX(ctx);
    int rc = check_misc(__func__, AXF_TYPE_Q8_0, W, x, y, rows, cols, row_bytes, true);
    if (rc) return rc;
    if (!rows || !cols) return AXF_OK;
    AXF_HIP(launch_gemv_q8w_f32(y, W, x, rows, cols / 32, (long)row_bytes, ctx->stream));
    return AXF_OK;
}

int axf_hip_gemv_q5_0_f32(axf_ctx* ctx, float* y, const void* W, const float* x, int rows,
                          int cols, size_t row_bytes) {
    AXF_CHECK_CTX(ctx);
    int rc = check_misc(__func__, AXF_TYPE_Q5_0, W, x, y, rows, cols, row_bytes, false);
    if (rc) return rc;
    if (!rows || !cols) return AXF_OK;
    AXF_HIP(launch_gemv_q5_0_f32(y, W, x, rows, cols / 32, (long)row_bytes, ctx->stream));
    return AXF_OK;
}

int axf_hip_gemv_f16_f32(axf_ctx* ctx, float* y, const void* W, const float* x, const float* b,
                         int rows, int cols) {
    AXF_CHECK_CTX(ctx);
    int rc = check_misc(__func__, AXF_TYPE_F16, W, x, y, rows, cols, (size_t)cols * 2, true);
    if (rc) return rc;
    if (!rows || !cols) return AXF_OK;
    AXF_HIP(launch_gemv_f16_f32(y, W, x, b, rows, cols, ctx->stream));
    return AXF_OK;
}

int axf_hip_gemm_misc_f32(axf_ctx* ctx, int qtype, float* Y, const void* W, const float* X,
                          int rows, int T, int cols, size_t row_bytes, int accumulate) {
    AXF_CHECK_CTX(ctx);
    const char* fn = "axf_hip_gemm_misc_f32";
    if (qtype != AXF_TYPE_Q8_0 && qtype != AXF_TYPE_Q5_0 && qtype != AXF_TYPE_F16)
        return fail(AXF_ERR_UNSUPPORTED, std::string(fn) + ": qtype must be Q8_0, Q5_0 or F16");
    if (T < 0 || T > 65535 * 16) return fail(AXF_ERR_INVALID_ARG, std::string(fn) + ": T out of range");
    if (cols % 32) return fail(AXF_ERR_INVALID_ARG, std::string(fn) + ": cols must be a multiple of 32");
    int rc = check_misc(fn, qtype, W, X, Y, rows, cols, qtype == AXF_TYPE_F16 ? (size_t)cols * 2 : row_bytes,
                        false);
    if (rc) return rc;
    if (qtype == AXF_TYPE_F16 && (row_bytes < (size_t)cols * 2 || row_bytes % 16))
        return fail(AXF_ERR_INVALID_ARG, std::string(fn) + ": F16 row_bytes must be >= 2*cols and a multiple of 16");
    if (!rows || !cols || !T) return AXF_OK;
    void* scratch = nullptr;  // the matrix-core form's hi/lo rows
    rc = ctx_scratch(ctx, gemm_misc_scratch_bytes(T, cols), &scratch);
    if (rc) return rc;
    AXF_HIP(launch_gemm_misc_f32(qtype, Y, W, X, rows, cols, (long)row_bytes, T, accumulate ? 1 : 0,
                                 ctx->stream, static_cast<float*>(scratch)));
    return AXF_OK;
}

int axf_hip_timer_start(axf_ctx* ctx) {
    AXF_CHECK_CTX(ctx);
    AXF_HIP(hipEventRecord(ctx->ev0, ctx->stream));
    return AXF_OK;
}

int axf_hip_timer_stop(axf_ctx* ctx, float* ms) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(ms, "null out");
    AXF_HIP(hipEventRecord(ctx->ev1, ctx->stream));
    AXF_HIP(hipEventSynchronize(ctx->ev1));
    AXF_HIP(hipEventElapsedTime(ms, ctx->ev0, ctx->ev1));
    return AXF_OK;
}

}  // extern "C"

// Capture n launches (launch(i, stream)) into one graph, replay it once
// untimed, then `reps` times between the context's two events.
template <class F>
static int bench_graph(axf_ctx* ctx, const char* fn, int n, int reps, float* ms, F launch) {
    hipStream_t st = ctx->stream;
    if (ctx->bench_eager) {  // direct launches: one warm-up pass, then reps passes
        hipError_t e = hipSuccess;
        for (int i = 0; i < n && e == hipSuccess; i++) e = launch(i, st);
        if (e == hipSuccess) e = hipEventRecord(ctx->ev0, st);
        for (int r = 0; r < reps && e == hipSuccess; r++)
            for (int i = 0; i < n && e == hipSuccess; i++) e = launch(i, st);
        if (e == hipSuccess) e = hipEventRecord(ctx->ev1, st);
        if (e == hipSuccess) e = hipEventSynchronize(ctx->ev1);
        if (e == hipSuccess) e = hipEventElapsedTime(ms, ctx->ev0, ctx->ev1);
        if (e != hipSuccess) return hip_fail(e, fn);
        return AXF_OK;
    }
    AXF_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    hipError_t e = hipSuccess;
    for (int i = 0; i < n && e == hipSuccess; i++) e = launch(i, st);
    hipGraph_t g = nullptr;
    hipError_t e2 = hipStreamEndCapture(st, &g);
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return hip_fail(e, fn);
    }
    if (e2 != hipSuccess) return hip_fail(e2, fn);
    hipGraphExec_t ex = nullptr;
    e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    if (e == hipSuccess) e = hipGraphLaunch(ex, st);
    if (e == hipSuccess) e = hipEventRecord(ctx->ev0, st);
    for (int r = 0; r < reps && e == hipSuccess; r++) e = hipGraphLaunch(ex, st);
    if (e == hipSuccess) e = hipEventRecord(ctx->ev1, st);
    if (e == hipSuccess) e = hipEventSynchronize(ctx->ev1);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, ctx->ev0, ctx->ev1);
    if (ex) (void)hipGraphExecDestroy(ex);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, fn);
    return AXF_OK;
}

extern "C" {

int axf_hip_bench_read(axf_ctx* ctx, const void* const* bufs, int n, size_t bytes, int unroll,
                       int wgs, int reps, float* ms) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(bufs && n > 0 && reps > 0 && ms && bytes >= 16 && bytes % 16 == 0 && wgs > 0,
                "bad arguments");
    AXF_REQUIRE(unroll == 1 || unroll == 2 || unroll == 4 || unroll == 8, "unroll must be 1/2/4/8");
    for (int i = 0; i < n; i++) AXF_REQUIRE(bufs[i] && aligned(bufs[i], 16), "buffer misaligned");
    void* sink = nullptr;
    int rc = ctx_scratch(ctx, 16, &sink);  // before any capture
    if (rc) return rc;
    return bench_graph(ctx, __func__, n, reps, ms, [&](int i, hipStream_t st) {
        return launch_stream_read(bufs[i], bytes, unroll, wgs, static_cast<uint32_t*>(sink), st);
    });
}

int axf_hip_bench_set_eager(axf_ctx* ctx, int eager) {
    AXF_CHECK_CTX(ctx);
    ctx->bench_eager = eager ? 1 : 0;
    return AXF_OK;
}

int axf_hip_bench_gemv(axf_ctx* ctx, int kind, float* y, const void* const* W_list, int n_w,
                       const void* x, int rows, int cols, size_t row_bytes, int reps, float* ms) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(kind >= 0 && kind <= 3 && W_list && n_w > 0 && reps > 0 && ms, "bad arguments");
    static const GemvKind kinds[4] = {GemvKind::Q4K_Q8, GemvKind::Q6K_Q8, GemvKind::Q4K_F32,
                                      GemvKind::Q6K_F32};
    const int qtype = (kind == 0 || kind == 2) ? AXF_TYPE_Q4_K : AXF_TYPE_Q6_K;
    for (int i = 0; i < n_w; i++) {
        int rc = check_gemv(__func__, qtype, W_list[i], x, y, rows, cols, row_bytes, kind >= 2);
        if (rc) return rc;
    }
    return bench_graph(ctx, __func__, n_w, reps, ms, [&](int i, hipStream_t st) {
        return launch_gemv(kinds[kind], y, W_list[i], x, rows, cols / QK_K, (long)row_bytes, 0, st);
    });
}

int axf_hip_bench_gemm(axf_ctx* ctx, int qtype, float* Y, const void* const* W_list, int n_w,
                       const void* XQ8, int rows, int T, int cols, size_t row_bytes, int path,
                       int reps, float* ms) {
    AXF_CHECK_CTX(ctx);
    AXF_REQUIRE(W_list && n_w > 0 && reps > 0 && ms && T > 0 && rows > 0 && cols > 0,
                "bad arguments");
    AXF_REQUIRE(qtype == AXF_TYPE_Q4_K || qtype == AXF_TYPE_Q6_K, "qtype must be Q4_K or Q6_K");
    AXF_REQUIRE(path >= 0 && path <= 3,
                "path must be 0 (auto), 1 (dot4), 2 (matrix cores) or 3 (matrix cores, streamed)");
    for (int i = 0; i < n_w; i++) {
        int rc = check_gemv(__func__, qtype, W_list[i], XQ8, Y, rows, cols, row_bytes, false);
        if (rc) return rc;
    }
    const size_t sb = gemm_scratch_bytes(qtype, (GemmPath)path, T, cols / QK_K, rows);
    void* scratch = nullptr;
    if (sb) {  // allocated before capture
        int rc = ctx_scratch(ctx, sb, &scratch);
        if (rc) return rc;
    }
    return bench_graph(ctx, __func__, n_w, reps, ms, [&](int i, hipStream_t st) {
        if (qtype == AXF_TYPE_Q6_K)
            return launch_gemm_q6k_q8(Y, W_list[i], XQ8, rows, T, cols / QK_K, (long)row_bytes,
                                      (GemmPath)path, scratch, st);
        return launch_gemm_q4k_q8(Y, W_list[i], XQ8, rows, T, cols / QK_K, (long)row_bytes,
                                  (GemmPath)path, scratch, st);
    });
}

size_t axf_row_bytes(int qtype, int64_t cols) {
    const int64_t nb = cols / QK_K;
    if (qtype == AXF_TYPE_Q4_K) return (size_t)nb * Q4K_BYTES;
    if (qtype == AXF_TYPE_Q6_K) return (size_t)nb * Q6K_BYTES;
    if (qtype == AXF_TYPE_F32) return (size_t)cols * 4;
    if (qtype == AXF_TYPE_F16) return (size_t)cols * 2;
    if (qtype == AXF_TYPE_Q8_0) return (size_t)(cols / 32) * 34;
    if (qtype == AXF_TYPE_Q5_0) return (size_t)(cols / 32) * 22;
    return 0;
}

int axf_rope_table(float* cos_t, float* sin_t, int hd, float theta, int max_pos) {
    AXF_REQUIRE(cos_t && sin_t && hd > 0 && hd % 2 == 0 && max_pos > 0, "bad arguments");
    // RopeCache::build (llama_model.cpp:1031-1043): float pow/cos/sin from libm.
    const int half = hd / 2;
    for (int p = 0; p < max_pos; p++) {
        for (int i = 0; i < half; i++) {
            const float freq = 1.f / std::pow(theta, (float)(2 * i) / (float)hd);
            const float angle = (float)p * freq;
            cos_t[(size_t)p * half + i] = std::cos(angle);
            sin_t[(size_t)p * half + i] = std::sin(angle);
        }
    }
    return AXF_OK;
}

}  // extern "C"
