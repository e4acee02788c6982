// ref_shim.cpp — C-ABI access to the reference's compiled x86 kernels.
//
// TEST INFRASTRUCTURE ONLY (checker and cpu_baseline).  oracle/Makefile
// compiles the reference kernel sources in place from
// /root/reference/src/backend/cpu_x86/kernels/*.cpp with the reference's own
// flags (src/backend/cpu_x86/CMakeLists.txt:7-39) and links them with this
// file into oracle/_ref/libaxf_ref.so.  This file only declares the
// reference's prototypes (as the reference itself does at
// src/models/llama_model.cpp:48-95) and forwards to them; the thread pool is
// the reference's header src/core/thread_pool.hpp, included where it lies.
#include <algorithm>
#include <chrono>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <memory>
#include <thread>
#include <vector>

#include "core/thread_pool.hpp"              // reference: src/core/thread_pool.hpp
#include "backend/cpu_x86/cpuid.hpp"         // reference: src/backend/cpu_x86/cpuid.hpp
#include "backend/cpu_x86/kernels/q8_block.hpp"  // reference: q8_block.hpp:8-15

namespace axonforge::cpu_x86 {
void gemv_q4k_avx2_range(float* y, const uint8_t* W, const float* x, int o_start, int o_end,
                         int in_dim, size_t row_bytes) noexcept;
void gemv_q6k_avx2_range(float* y, const uint8_t* W, const float* x, int o_start, int o_end,
                         int in_dim, size_t row_bytes) noexcept;
void quantize_q8_avx2(block_q8_0* y, const float* x, int k) noexcept;
void gemv_q4k_q8_avx2_range(float* y, const uint8_t* W, const block_q8_0* xq8, int o_start,
                            int o_end, int in_dim, size_t row_bytes) noexcept;
void gemv_q4k_q8_avxvnni_range(float* y, const uint8_t* W, const block_q8_0* xq8, int o_start,
                               int o_end, int in_dim, size_t row_bytes) noexcept;
void gemm_q4k_q8_avx2_range(float* Y, const uint8_t* W, const block_q8_0* XQ8, int M, int T,
                            int K, size_t row_bytes, int o_start, int o_end) noexcept;
void gemm_q4k_q8_avxvnni_range(float* Y, const uint8_t* W, const block_q8_0* XQ8, int M, int T,
                               int K, size_t row_bytes, int o_start, int o_end) noexcept;
void gemv_q6k_q8_avx2_range(float* y, const uint8_t* W, const block_q8_0* xq8, int o_start,
                            int o_end, int in_dim, size_t row_bytes) noexcept;
void repack_q4k_8rows(uint8_t* dst, const uint8_t* src, int nrows, int ncols) noexcept;
void gemv_q4k_r8_avx2_range(float* y, const uint8_t* R8, const block_q8_0* xq8, int o_start,
                            int o_end, int in_dim) noexcept;
void gemv_q4k_r8_avxvnni_range(float* y, const uint8_t* R8, const block_q8_0* xq8, int o_start,
                               int o_end, int in_dim) noexcept;
}  // namespace axonforge::cpu_x86

namespace cx = axonforge::cpu_x86;

extern "C" {

int ref_has_avxvnni(void) { return cx::cpu_features().avxvnni ? 1 : 0; }
int ref_has_avx2(void) { return cx::cpu_features().avx2 ? 1 : 0; }

void ref_gemv_q4k_f32(float* y, const uint8_t* W, const float* x, int o0, int o1, int in_dim,
                      size_t rb) {
    cx::gemv_q4k_avx2_range(y, W, x, o0, o1, in_dim, rb);
}
void ref_gemv_q6k_f32(float* y, const uint8_t* W, const float* x, int o0, int o1, int in_dim,
                      size_t rb) {
    cx::gemv_q6k_avx2_range(y, W, x, o0, o1, in_dim, rb);
}
void ref_quantize_q8_0(void* y, const float* x, int k) {
    cx::quantize_q8_avx2(static_cast<block_q8_0*>(y), x, k);
}
void ref_gemv_q4k_q8(float* y, const uint8_t* W, const void* xq8, int o0, int o1, int in_dim,
                     size_t rb, int vnni) {
    auto* xq = static_cast<const block_q8_0*>(xq8);
    if (vnni)
        cx::gemv_q4k_q8_avxvnni_range(y, W, xq, o0, o1, in_dim, rb);
    else
        cx::gemv_q4k_q8_avx2_range(y, W, xq, o0, o1, in_dim, rb);
}
void ref_repack_q4k_r8(uint8_t* dst, const uint8_t* src, int nrows, int ncols) {
    cx::repack_q4k_8rows(dst, src, nrows, ncols);
}
void ref_gemv_q4k_r8(float* y, const uint8_t* R8, const void* xq8, int o0, int o1, int in_dim,
                     int vnni) {
    auto* xq = static_cast<const block_q8_0*>(xq8);
    if (vnni)
        cx::gemv_q4k_r8_avxvnni_range(y, R8, xq, o0, o1, in_dim);
    else
        cx::gemv_q4k_r8_avx2_range(y, R8, xq, o0, o1, in_dim);
}
void ref_gemv_q6k_q8(float* y, const uint8_t* W, const void* xq8, int o0, int o1, int in_dim,
                     size_t rb) {
    cx::gemv_q6k_q8_avx2_range(y, W, static_cast<const block_q8_0*>(xq8), o0, o1, in_dim, rb);
}
void ref_gemm_q4k_q8(float* Y, const uint8_t* W, const void* XQ8, int M, int T, int K, size_t rb,
                     int o0, int o1, int vnni) {
    auto* xq = static_cast<const block_q8_0*>(XQ8);
    if (vnni)
        cx::gemm_q4k_q8_avxvnni_range(Y, W, xq, M, T, K, rb, o0, o1);
    else
        cx::gemm_q4k_q8_avx2_range(Y, W, xq, M, T, K, rb, o0, o1);
}

// ---------------------------------------------------------------------------
// CPU baseline timing: the reference decode-path GEMV as gemv_wt_q8 runs it
// (llama_model.cpp:767-831) — Q8_0 quantize of x, then the r8 kernel (VNNI
// when CPUID reports AVX-VNNI, else AVX2) for Q4_K, or the 4-row Q6_K kernel,
// split over ThreadPool::parallel_for with n_threads = min(16, nproc) and the
// reference's CPU pinning (llama_model.cpp:1524-1557).
//
// W_copies: n_copies weight buffers (native layout for Q6_K, r8 layout for
// Q4_K) that are rotated between calls so the weights stream from DRAM.
// Returns the median seconds per call over `iters` timed calls after 3
// warm-ups; *threads_used receives the thread count.
// ---------------------------------------------------------------------------
double ref_time_decode_gemv(int qtype, const uint8_t* const* W_copies, int n_copies, int rows,
                            int cols, const float* x, float* y, int iters, int n_threads,
                            int* threads_used) {
    if (n_threads <= 0)
        n_threads = std::min(16, (int)std::thread::hardware_concurrency());
    if (threads_used) *threads_used = n_threads;
    const int nw = n_threads - 1;
    // Save the caller's affinity and restore it afterwards, as
    // llama_generate_cpu_impl does around its pinned region (:1531-1537, :1626-1628).
    cpu_set_t orig_aff;
    sched_getaffinity(0, sizeof(orig_aff), &orig_aff);
    std::unique_ptr<axonforge::ThreadPool> pool;
    if (nw > 0) {
        pool = std::make_unique<axonforge::ThreadPool>(nw);
        axonforge::ThreadPool::pin_caller(nw);
    }
    std::vector<block_q8_0> xq8((size_t)cols / 32);
    const bool vnni = cx::cpu_features().avxvnni;
    const bool q6 = (qtype == 14);
    const size_t rb = (size_t)(cols / 256) * (q6 ? 210 : 144);

    auto one = [&](const uint8_t* W) {
        cx::quantize_q8_avx2(xq8.data(), x, cols);
        const block_q8_0* xq = xq8.data();
        if (q6) {
            auto fn = [&](int s, int e) { cx::gemv_q6k_q8_avx2_range(y, W, xq, s, e, cols, rb); };
            if (pool && rows >= 32) pool->parallel_for(rows, fn); else fn(0, rows);
        } else {
            const int n8 = rows / 8;
            auto fn = [&](int gs, int ge) {
                if (vnni)
                    cx::gemv_q4k_r8_avxvnni_range(y, W, xq, gs * 8, ge * 8, cols);
                else
                    cx::gemv_q4k_r8_avx2_range(y, W, xq, gs * 8, ge * 8, cols);
            };
            if (pool && n8 >= 2) pool->parallel_for(n8, fn); else fn(0, n8);
        }
    };
    for (int i = 0; i < 3; i++) one(W_copies[i % n_copies]);
    std::vector<double> t(iters);
    for (int i = 0; i < iters; i++) {
        const uint8_t* W = W_copies[(i + 3) % n_copies];
        auto t0 = std::chrono::steady_clock::now();
        one(W);
        auto t1 = std::chrono::steady_clock::now();
        t[i] = std::chrono::duration<double>(t1 - t0).count();
    }
    pool.reset();
    sched_setaffinity(0, sizeof(orig_aff), &orig_aff);
    std::sort(t.begin(), t.end());
    return t[iters / 2];
}

}  // extern "C"
