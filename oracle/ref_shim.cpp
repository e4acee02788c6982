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
#include <cmath>
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
void gemv_f16_avx2_range(float* y, const uint16_t* W, const float* x, const float* b,
                         int o_start, int o_end, int in) noexcept;
void gemv_q4k_r8_avx2_range(float* y, const uint8_t* R8, const block_q8_0* xq8, int o_start,
                            int o_end, int in_dim) noexcept;
void gemv_q4k_r8_avxvnni_range(float* y, const uint8_t* R8, const block_q8_0* xq8, int o_start,
                               int o_end, int in_dim) noexcept;
}  // namespace axonforge::cpu_x86

namespace cx = axonforge::cpu_x86;

extern "C" {

int ref_has_avxvnni(void) { return cx::cpu_features().avxvnni ? 1 : 0; }

void ref_gemv_f16_f32(float* y, const uint16_t* W, const float* x, const float* b, int o0,
                      int o1, int in_dim) {
    cx::gemv_f16_avx2_range(y, W, x, b, o0, o1, in_dim);
}
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

// ---------------------------------------------------------------------------
// CPU baselines of the other configurations, each with the reference's
// dispatch on its ThreadPool (n_threads = min(16, nproc), pinned as above),
// weights rotated over n_copies buffers; median seconds per call over `iters`
// timed calls after 3 warm-ups.
//   ref_time_gemv_f32: gemv_wt (llama_model.cpp:670-700) for Q4_K / Q6_K with
//     fp32 activations: parallel_for over rows (>= 32) of gemv_q4k_avx2_range /
//     gemv_q6k_avx2_range (config 1).
//   ref_time_gemm_q4k: gemm_wt_q8's Q4_K branch (llama_model.cpp:837-858):
//     parallel_for over rows (>= 32) of gemm_q4k_q8_{avxvnni,avx2}_range on T
//     Q8_0 token rows already quantised (config 4).
//   ref_time_head_argmax: the decode GEMV of ref_time_decode_gemv for a Q6_K
//     head, then the greedy pick std::max_element (sample, :1466-1471)
//     (config 2).
// ---------------------------------------------------------------------------
}  // extern "C"

namespace {

template <class F>
double time_median(const uint8_t* const* W_copies, int n_copies, int iters, F&& one) {
    for (int i = 0; i < 3; i++) one(W_copies[i % n_copies]);
    std::vector<double> t((size_t)std::max(iters, 1));
    for (int i = 0; i < iters; i++) {
        const uint8_t* W = W_copies[(i + 3) % n_copies];
        auto t0 = std::chrono::steady_clock::now();
        one(W);
        auto t1 = std::chrono::steady_clock::now();
        t[i] = std::chrono::duration<double>(t1 - t0).count();
    }
    std::sort(t.begin(), t.begin() + iters);
    return iters > 0 ? t[iters / 2] : 0.0;
}

struct PinnedPool {
    cpu_set_t orig;
    std::unique_ptr<axonforge::ThreadPool> pool;
    explicit PinnedPool(int& n_threads) {
        if (n_threads <= 0) n_threads = std::min(16, (int)std::thread::hardware_concurrency());
        sched_getaffinity(0, sizeof(orig), &orig);
        if (n_threads > 1) {
            pool = std::make_unique<axonforge::ThreadPool>(n_threads - 1);
            axonforge::ThreadPool::pin_caller(n_threads - 1);
        }
    }
    ~PinnedPool() {
        pool.reset();
        sched_setaffinity(0, sizeof(orig), &orig);
    }
};

}  // namespace

extern "C" {

double ref_time_gemv_f32(int qtype, const uint8_t* const* W_copies, int n_copies, int rows,
                         int cols, const float* x, float* y, int iters, int n_threads,
                         int* threads_used) {
    PinnedPool pp(n_threads);
    if (threads_used) *threads_used = n_threads;
    const bool q6 = (qtype == 14);
    const size_t rb = (size_t)(cols / 256) * (q6 ? 210 : 144);
    return time_median(W_copies, n_copies, iters, [&](const uint8_t* W) {
        auto fn = [&](int s, int e) {
            if (q6)
                cx::gemv_q6k_avx2_range(y, W, x, s, e, cols, rb);
            else
                cx::gemv_q4k_avx2_range(y, W, x, s, e, cols, rb);
        };
        if (pp.pool && rows >= 32) pp.pool->parallel_for(rows, fn); else fn(0, rows);
    });
}

double ref_time_gemm_q4k(const uint8_t* const* W_copies, int n_copies, int rows, int cols,
                         const void* XQ8, int T, float* Y, int iters, int n_threads,
                         int* threads_used) {
    PinnedPool pp(n_threads);
    if (threads_used) *threads_used = n_threads;
    const size_t rb = (size_t)(cols / 256) * 144;
    const bool vnni = cx::cpu_features().avxvnni;
    auto* xq = static_cast<const block_q8_0*>(XQ8);
    return time_median(W_copies, n_copies, iters, [&](const uint8_t* W) {
        auto fn = [&](int s, int e) {
            if (vnni)
                cx::gemm_q4k_q8_avxvnni_range(Y, W, xq, rows, T, cols, rb, s, e);
            else
                cx::gemm_q4k_q8_avx2_range(Y, W, xq, rows, T, cols, rb, s, e);
        };
        if (pp.pool && rows >= 32) pp.pool->parallel_for(rows, fn); else fn(0, rows);
    });
}

double ref_time_head_argmax(const uint8_t* const* W_copies, int n_copies, int rows, int cols,
                            const float* x, float* y, int iters, int n_threads, int* threads_used,
                            int* argmax) {
    PinnedPool pp(n_threads);
    if (threads_used) *threads_used = n_threads;
    const size_t rb = (size_t)(cols / 256) * 210;
    std::vector<block_q8_0> xq8((size_t)cols / 32);
    int best = 0;
    const double t = time_median(W_copies, n_copies, iters, [&](const uint8_t* W) {
        cx::quantize_q8_avx2(xq8.data(), x, cols);
        const block_q8_0* xq = xq8.data();
        auto fn = [&](int s, int e) { cx::gemv_q6k_q8_avx2_range(y, W, xq, s, e, cols, rb); };
        if (pp.pool && rows >= 32) pp.pool->parallel_for(rows, fn); else fn(0, rows);
        best = (int)(std::max_element(y, y + rows) - y);
    });
    if (argmax) *argmax = best;
    return t;
}

// ---------------------------------------------------------------------------
// CPU baseline for the whole decode step: llama_forward_token
// (llama_model.cpp:1207-1333) with the reference's dispatch — Q8_0 quantize,
// r8 Q4_K GEMV (VNNI or AVX2 by CPUID) over 8-row groups, Q6_K 4-row GEMV,
// gate+up+SwiGLU fused in one parallel_for (Fusion C, :1284-1314) — on the
// reference ThreadPool.  The ops that live as static functions in
// llama_model.cpp (RMSNorm, RoPE, attention, SwiGLU, embedding dequant) come
// from the oracle's restatement of them (axf_oracle.c), single-threaded as in
// the reference.  Every timed step runs at position `pos` (rows below pos of
// the caller's KV cache must be filled; row pos is rewritten).  Returns the
// median seconds per step.
// ---------------------------------------------------------------------------
}  // extern "C"

#include "axf_oracle.h"

namespace {

struct WtR {
    const orc_wt* w;
    std::vector<uint8_t> r8;  // repacked copy when Q4_K with rows % 8 == 0
};

WtR make_wt(const orc_wt* w, int rows, int cols) {
    WtR r{w, {}};
    if (w->type == ORC_TYPE_Q4_K && rows % 8 == 0) {
        r.r8.resize((size_t)(rows / 8) * (cols / 256) * 1152);
        cx::repack_q4k_8rows(r.r8.data(), w->data, rows, cols);
    }
    return r;
}

// gemv_wt_q8 (llama_model.cpp:767-831)
void gemv_wt_q8(float* y, const WtR& W, const block_q8_0* xq8, int out, int in,
                axonforge::ThreadPool* pool, bool vnni) {
    if (W.w->type == ORC_TYPE_Q4_K && !W.r8.empty()) {
        const uint8_t* R8 = W.r8.data();
        const int n8 = out / 8;
        auto fn = [&](int gs, int ge) {
            if (vnni)
                cx::gemv_q4k_r8_avxvnni_range(y, R8, xq8, gs * 8, ge * 8, in);
            else
                cx::gemv_q4k_r8_avx2_range(y, R8, xq8, gs * 8, ge * 8, in);
        };
        if (pool && n8 >= 2) pool->parallel_for(n8, fn); else fn(0, n8);
        return;
    }
    const size_t rb = (size_t)(in / 256) * (W.w->type == ORC_TYPE_Q6_K ? 210 : 144);
    auto fn = [&](int s, int e) {
        if (W.w->type == ORC_TYPE_Q6_K)
            cx::gemv_q6k_q8_avx2_range(y, W.w->data, xq8, s, e, in, rb);
        else if (vnni)
            cx::gemv_q4k_q8_avxvnni_range(y, W.w->data, xq8, s, e, in, rb);
        else
            cx::gemv_q4k_q8_avx2_range(y, W.w->data, xq8, s, e, in, rb);
    };
    if (pool && out >= 32) pool->parallel_for(out, fn); else fn(0, out);
}

}  // namespace

extern "C" double ref_time_decode_step(const orc_model* m, float* kv_k, float* kv_v, int pos,
                                       int warmup, int steps, int n_threads, int* threads_used,
                                       int* last_token) {
    if (n_threads <= 0) n_threads = std::min(16, (int)std::thread::hardware_concurrency());
    if (threads_used) *threads_used = n_threads;
    const int E = m->n_embd, H = m->n_heads, KVH = m->n_kv_heads, HD = E / H, FD = m->ffn_dim;
    const int kve = KVH * HD, L = m->n_layer, NC = m->n_ctx;
    const bool vnni = cx::cpu_features().avxvnni;

    // build_weights + repack_q4k_if_avx2 (llama_model.cpp:963-1019), untimed
    std::vector<WtR> wq, wk, wv, wo, wg, wu, wd;
    for (int l = 0; l < L; l++) {
        const orc_layer& lw = m->layers[l];
        wq.push_back(make_wt(&lw.wq, H * HD, E));
        wk.push_back(make_wt(&lw.wk, kve, E));
        wv.push_back(make_wt(&lw.wv, kve, E));
        wo.push_back(make_wt(&lw.wo, E, H * HD));
        wg.push_back(make_wt(&lw.wgate, FD, E));
        wu.push_back(make_wt(&lw.wup, FD, E));
        wd.push_back(make_wt(&lw.wdown, E, FD));
    }
    WtR head = make_wt(&m->output, m->n_vocab, E);

    cpu_set_t orig_aff;
    sched_getaffinity(0, sizeof(orig_aff), &orig_aff);
    const int nw = n_threads - 1;
    std::unique_ptr<axonforge::ThreadPool> pool;
    if (nw > 0) {
        pool = std::make_unique<axonforge::ThreadPool>(nw);
        axonforge::ThreadPool::pin_caller(nw);
    }
    std::vector<float> x(E), xb(E), q(H * HD), k(kve), v(kve), attn(NC), ao(E), gate(FD), up(FD),
        ffn(E), logits(m->n_vocab), rc((size_t)NC * HD / 2), rs((size_t)NC * HD / 2);
    std::vector<block_q8_0> xq8((size_t)std::max(E, FD) / 32);
    orc_rope_table(rc.data(), rs.data(), HD, m->rope_theta, NC);
    int token = 1;

    auto step = [&]() {
        const size_t rbe = (size_t)(E / 256) * (m->tok_embd.type == ORC_TYPE_Q6_K ? 210 : 144);
        if (m->tok_embd.type == ORC_TYPE_Q6_K)
            orc_dequant_q6k(x.data(), m->tok_embd.data + (size_t)token * rbe, E / 256);
        else
            orc_dequant_q4k(x.data(), m->tok_embd.data + (size_t)token * rbe, E / 256);
        block_q8_0* xq = xq8.data();
        for (int l = 0; l < L; l++) {
            const orc_layer& lw = m->layers[l];
            float* kc = kv_k + (size_t)l * NC * kve;
            float* vc = kv_v + (size_t)l * NC * kve;
            orc_rmsnorm(xb.data(), x.data(), lw.attn_norm, E, m->rms_eps);
            cx::quantize_q8_avx2(xq, xb.data(), E);
            gemv_wt_q8(q.data(), wq[l], xq, H * HD, E, pool.get(), vnni);
            gemv_wt_q8(k.data(), wk[l], xq, kve, E, pool.get(), vnni);
            gemv_wt_q8(v.data(), wv[l], xq, kve, E, pool.get(), vnni);
            for (int i = 0; lw.bq && i < H * HD; i++) q[i] += lw.bq[i];
            for (int i = 0; lw.bk && i < kve; i++) k[i] += lw.bk[i];
            for (int i = 0; lw.bv && i < kve; i++) v[i] += lw.bv[i];
            orc_rope(q.data(), q.data(), pos, H, HD, rc.data(), rs.data());
            orc_rope(kc + (size_t)pos * kve, k.data(), pos, KVH, HD, rc.data(), rs.data());
            std::memcpy(vc + (size_t)pos * kve, v.data(), sizeof(float) * kve);
            orc_attention(ao.data(), q.data(), kc, vc, pos + 1, H, KVH, HD, attn.data());
            cx::quantize_q8_avx2(xq, ao.data(), E);
            gemv_wt_q8(xb.data(), wo[l], xq, E, E, pool.get(), vnni);
            for (int i = 0; i < E; i++) x[i] += xb[i];
            orc_rmsnorm(xb.data(), x.data(), lw.ffn_norm, E, m->rms_eps);
            cx::quantize_q8_avx2(xq, xb.data(), E);
            if (!wg[l].r8.empty() && !wu[l].r8.empty() && pool) {
                const uint8_t* R8g = wg[l].r8.data();
                const uint8_t* R8u = wu[l].r8.data();
                pool->parallel_for(FD / 8, [&](int gs, int ge) {
                    const int s0 = gs * 8, e0 = ge * 8;
                    if (vnni) {
                        cx::gemv_q4k_r8_avxvnni_range(gate.data(), R8g, xq, s0, e0, E);
                        cx::gemv_q4k_r8_avxvnni_range(up.data(), R8u, xq, s0, e0, E);
                    } else {
                        cx::gemv_q4k_r8_avx2_range(gate.data(), R8g, xq, s0, e0, E);
                        cx::gemv_q4k_r8_avx2_range(up.data(), R8u, xq, s0, e0, E);
                    }
                    orc_swiglu(gate.data() + s0, up.data() + s0, e0 - s0);
                });
            } else {
                gemv_wt_q8(gate.data(), wg[l], xq, FD, E, pool.get(), vnni);
                gemv_wt_q8(up.data(), wu[l], xq, FD, E, pool.get(), vnni);
                orc_swiglu(gate.data(), up.data(), FD);
            }
            cx::quantize_q8_avx2(xq, gate.data(), FD);
            gemv_wt_q8(ffn.data(), wd[l], xq, E, FD, pool.get(), vnni);
            for (int i = 0; i < E; i++) x[i] += ffn[i];
        }
        orc_rmsnorm(x.data(), x.data(), m->output_norm, E, m->rms_eps);
        cx::quantize_q8_avx2(xq, x.data(), E);
        gemv_wt_q8(logits.data(), head, xq, m->n_vocab, E, pool.get(), vnni);
        token = orc_argmax(logits.data(), m->n_vocab);
    };

    for (int i = 0; i < warmup; i++) step();
    std::vector<double> t((size_t)std::max(steps, 1));
    for (int i = 0; i < steps; i++) {
        auto t0 = std::chrono::steady_clock::now();
        step();
        auto t1 = std::chrono::steady_clock::now();
        t[i] = std::chrono::duration<double>(t1 - t0).count();
    }
    pool.reset();
    sched_setaffinity(0, sizeof(orig_aff), &orig_aff);
    if (last_token) *last_token = token;
    std::sort(t.begin(), t.begin() + steps);
    return steps > 0 ? t[steps / 2] : 0.0;
}

// ---------------------------------------------------------------------------
// Greedy generation of llama_generate_cpu_impl (llama_model.cpp:1502-1631)
// with temperature 0, no repetition penalty and no EOS stop, on the
// reference's compiled kernels: the prompt (used as given: the caller starts
// it with BOS) prefilled as one llama_forward_batch (:1339-1462: Q8_0 rows,
// the Q4_K GEMM over all tokens, Q6_K per token, causal attention of every
// row), then llama_forward_token per generated token (:1207-1333, the r8 /
// 4-row Q8_0 GEMVs and the fused gate+up) - the GEMMs and GEMVs split over
// the reference ThreadPool by rows, which does not change any result (each
// output is computed by one thread).  The glue ops are the oracle's
// restatement.  out_tokens[i] = the i-th generated id; out_margins[i] = the
// top-1 minus top-2 logit it was taken from.  Returns the number generated
// (stops at the context end).
// ---------------------------------------------------------------------------
namespace {

void gemm_wt_q8_ref(float* Y, const WtR& W, const block_q8_0* XQ8, int M, int T, int K,
                    axonforge::ThreadPool* pool, bool vnni) {
    const size_t rb = (size_t)(K / 256) * (W.w->type == ORC_TYPE_Q6_K ? 210 : 144);
    auto fn = [&](int s, int e) {
        if (W.w->type == ORC_TYPE_Q6_K) {
            for (int t = 0; t < T; t++)
                cx::gemv_q6k_q8_avx2_range(Y + (size_t)t * M, W.w->data, XQ8 + (size_t)t * (K / 32),
                                           s, e, K, rb);
        } else if (vnni) {
            cx::gemm_q4k_q8_avxvnni_range(Y, W.w->data, XQ8, M, T, K, rb, s, e);
        } else {
            cx::gemm_q4k_q8_avx2_range(Y, W.w->data, XQ8, M, T, K, rb, s, e);
        }
    };
    if (pool && M >= 32) pool->parallel_for(M, fn); else fn(0, M);
}

}  // namespace

extern "C" int ref_generate_greedy(const orc_model* m, const int32_t* prompt, int n_prompt,
                                   int n_gen, int n_threads, int32_t* out_tokens,
                                   float* out_margins, int top_k, int32_t* top_ids,
                                   float* top_vals) {
    if (n_threads <= 0) n_threads = std::min(16, (int)std::thread::hardware_concurrency());
    const int E = m->n_embd, H = m->n_heads, KVH = m->n_kv_heads, HD = E / H, FD = m->ffn_dim;
    const int kve = KVH * HD, L = m->n_layer, NC = m->n_ctx, V = m->n_vocab, T = n_prompt;
    if (T < 1 || T > NC) return 0;
    const bool vnni = cx::cpu_features().avxvnni;
    std::vector<WtR> wq, wk, wv, wo, wg, wu, wd;
    for (int l = 0; l < L; l++) {
        const orc_layer& lw = m->layers[l];
        wq.push_back(make_wt(&lw.wq, H * HD, E));
        wk.push_back(make_wt(&lw.wk, kve, E));
        wv.push_back(make_wt(&lw.wv, kve, E));
        wo.push_back(make_wt(&lw.wo, E, H * HD));
        wg.push_back(make_wt(&lw.wgate, FD, E));
        wu.push_back(make_wt(&lw.wup, FD, E));
        wd.push_back(make_wt(&lw.wdown, E, FD));
    }
    WtR head = make_wt(&m->output, V, E);
    cpu_set_t orig_aff;
    sched_getaffinity(0, sizeof(orig_aff), &orig_aff);
    const int nw = n_threads - 1;
    std::unique_ptr<axonforge::ThreadPool> pool;
    if (nw > 0) {
        pool = std::make_unique<axonforge::ThreadPool>(nw);
        axonforge::ThreadPool::pin_caller(nw);
    }
    std::vector<float> kv_k((size_t)L * NC * kve), kv_v(kv_k.size());
    std::vector<float> rc((size_t)NC * HD / 2), rs(rc.size()), logits(V);
    orc_rope_table(rc.data(), rs.data(), HD, m->rope_theta, NC);
    const size_t rbe = (size_t)(E / 256) * (m->tok_embd.type == ORC_TYPE_Q6_K ? 210 : 144);
    auto embed = [&](float* out, int tok) {
        if (m->tok_embd.type == ORC_TYPE_Q6_K)
            orc_dequant_q6k(out, m->tok_embd.data + (size_t)tok * rbe, E / 256);
        else
            orc_dequant_q4k(out, m->tok_embd.data + (size_t)tok * rbe, E / 256);
    };
    auto add_rows = [](float* y, const float* b, int rows, int n) {
        if (!b) return;
        for (int t = 0; t < rows; t++)
            for (int i = 0; i < n; i++) y[(size_t)t * n + i] += b[i];
    };

    // ---- batched prefill (llama_forward_batch) ----
    std::vector<float> X((size_t)T * E), XB((size_t)T * E), Q((size_t)T * H * HD), K((size_t)T * kve),
        Vv((size_t)T * kve), AO((size_t)T * E), GATE((size_t)T * FD), UP((size_t)T * FD),
        FFN((size_t)T * E);
    std::vector<block_q8_0> XQE((size_t)T * (E / 32)), XQF((size_t)T * (FD / 32));
    std::vector<float> attn_scratch((size_t)(nw + 1) * NC);
    for (int t = 0; t < T; t++) embed(X.data() + (size_t)t * E, prompt[t]);
    for (int l = 0; l < L; l++) {
        const orc_layer& lw = m->layers[l];
        float* kc = kv_k.data() + (size_t)l * NC * kve;
        float* vc = kv_v.data() + (size_t)l * NC * kve;
        for (int t = 0; t < T; t++) {
            orc_rmsnorm(XB.data() + (size_t)t * E, X.data() + (size_t)t * E, lw.attn_norm, E, m->rms_eps);
            cx::quantize_q8_avx2(XQE.data() + (size_t)t * (E / 32), XB.data() + (size_t)t * E, E);
        }
        gemm_wt_q8_ref(Q.data(), wq[l], XQE.data(), H * HD, T, E, pool.get(), vnni);
        gemm_wt_q8_ref(K.data(), wk[l], XQE.data(), kve, T, E, pool.get(), vnni);
        gemm_wt_q8_ref(Vv.data(), wv[l], XQE.data(), kve, T, E, pool.get(), vnni);
        add_rows(Q.data(), lw.bq, T, H * HD);
        add_rows(K.data(), lw.bk, T, kve);
        add_rows(Vv.data(), lw.bv, T, kve);
        for (int t = 0; t < T; t++) {
            orc_rope(Q.data() + (size_t)t * H * HD, Q.data() + (size_t)t * H * HD, t, H, HD, rc.data(),
                     rs.data());
            orc_rope(kc + (size_t)t * kve, K.data() + (size_t)t * kve, t, KVH, HD, rc.data(), rs.data());
            std::memcpy(vc + (size_t)t * kve, Vv.data() + (size_t)t * kve, sizeof(float) * kve);
        }
        // causal attention: row t over positions 0..t (rows split over threads;
        // each row's arithmetic is the sequential one of :1410-1426)
        auto att = [&](int s, int e) {
            static thread_local std::vector<float> scratch;
            if ((int)scratch.size() < NC) scratch.resize(NC);
            for (int t = s; t < e; t++)
                orc_attention(AO.data() + (size_t)t * E, Q.data() + (size_t)t * H * HD, kc, vc, t + 1,
                              H, KVH, HD, scratch.data());
        };
        if (pool) pool->parallel_for(T, att); else att(0, T);
        for (int t = 0; t < T; t++)
            cx::quantize_q8_avx2(XQE.data() + (size_t)t * (E / 32), AO.data() + (size_t)t * E, E);
        gemm_wt_q8_ref(XB.data(), wo[l], XQE.data(), E, T, E, pool.get(), vnni);
        for (size_t i = 0; i < (size_t)T * E; i++) X[i] += XB[i];
        for (int t = 0; t < T; t++) {
            orc_rmsnorm(XB.data() + (size_t)t * E, X.data() + (size_t)t * E, lw.ffn_norm, E, m->rms_eps);
            cx::quantize_q8_avx2(XQE.data() + (size_t)t * (E / 32), XB.data() + (size_t)t * E, E);
        }
        gemm_wt_q8_ref(GATE.data(), wg[l], XQE.data(), FD, T, E, pool.get(), vnni);
        gemm_wt_q8_ref(UP.data(), wu[l], XQE.data(), FD, T, E, pool.get(), vnni);
        for (int t = 0; t < T; t++) {
            orc_swiglu(GATE.data() + (size_t)t * FD, UP.data() + (size_t)t * FD, FD);
            cx::quantize_q8_avx2(XQF.data() + (size_t)t * (FD / 32), GATE.data() + (size_t)t * FD, FD);
        }
        gemm_wt_q8_ref(FFN.data(), wd[l], XQF.data(), E, T, FD, pool.get(), vnni);
        for (size_t i = 0; i < (size_t)T * E; i++) X[i] += FFN[i];
    }
    std::vector<float> x(X.begin() + (size_t)(T - 1) * E, X.begin() + (size_t)T * E);
    std::vector<block_q8_0> xq8((size_t)std::max(E, FD) / 32);
    orc_rmsnorm(x.data(), x.data(), m->output_norm, E, m->rms_eps);
    cx::quantize_q8_avx2(xq8.data(), x.data(), E);
    gemv_wt_q8(logits.data(), head, xq8.data(), V, E, pool.get(), vnni);
    X.clear(); XB.clear(); Q.clear(); K.clear(); Vv.clear(); AO.clear(); GATE.clear(); UP.clear();
    FFN.clear();

    // ---- decode loop (llama_forward_token per generated token) ----
    std::vector<float> xb(E), q(H * HD), k(kve), v(kve), attn(NC), ao(E), gate(FD), up(FD), ffn(E);
    int n = 0, n_past = T;
    for (int step = 0; step < n_gen; step++) {
        if (n_past >= NC) break;
        const int tok = orc_argmax(logits.data(), V);
        out_tokens[n] = tok;
        out_margins[n] = orc_top2_margin(logits.data(), V);
        if (top_k > 0 && top_ids && top_vals) {
            // the top_k logits of this step, largest first (ties: lower id first)
            std::vector<int32_t> idx(V);
            for (int i = 0; i < V; i++) idx[i] = i;
            const int kk = std::min(top_k, V);
            std::partial_sort(idx.begin(), idx.begin() + kk, idx.end(), [&](int32_t a, int32_t b) {
                return logits[a] > logits[b] || (logits[a] == logits[b] && a < b);
            });
            for (int i = 0; i < kk; i++) {
                top_ids[(size_t)n * top_k + i] = idx[i];
                top_vals[(size_t)n * top_k + i] = logits[idx[i]];
            }
        }
        n++;
        const int pos = n_past;
        embed(x.data(), tok);
        block_q8_0* xq = xq8.data();
        for (int l = 0; l < L; l++) {
            const orc_layer& lw = m->layers[l];
            float* kc = kv_k.data() + (size_t)l * NC * kve;
            float* vc = kv_v.data() + (size_t)l * NC * kve;
            orc_rmsnorm(xb.data(), x.data(), lw.attn_norm, E, m->rms_eps);
            cx::quantize_q8_avx2(xq, xb.data(), E);
            gemv_wt_q8(q.data(), wq[l], xq, H * HD, E, pool.get(), vnni);
            gemv_wt_q8(k.data(), wk[l], xq, kve, E, pool.get(), vnni);
            gemv_wt_q8(v.data(), wv[l], xq, kve, E, pool.get(), vnni);
            for (int i = 0; lw.bq && i < H * HD; i++) q[i] += lw.bq[i];
            for (int i = 0; lw.bk && i < kve; i++) k[i] += lw.bk[i];
            for (int i = 0; lw.bv && i < kve; i++) v[i] += lw.bv[i];
            orc_rope(q.data(), q.data(), pos, H, HD, rc.data(), rs.data());
            orc_rope(kc + (size_t)pos * kve, k.data(), pos, KVH, HD, rc.data(), rs.data());
            std::memcpy(vc + (size_t)pos * kve, v.data(), sizeof(float) * kve);
            orc_attention(ao.data(), q.data(), kc, vc, pos + 1, H, KVH, HD, attn.data());
            cx::quantize_q8_avx2(xq, ao.data(), E);
            gemv_wt_q8(xb.data(), wo[l], xq, E, E, pool.get(), vnni);
            for (int i = 0; i < E; i++) x[i] += xb[i];
            orc_rmsnorm(xb.data(), x.data(), lw.ffn_norm, E, m->rms_eps);
            cx::quantize_q8_avx2(xq, xb.data(), E);
            gemv_wt_q8(gate.data(), wg[l], xq, FD, E, pool.get(), vnni);
            gemv_wt_q8(up.data(), wu[l], xq, FD, E, pool.get(), vnni);
            orc_swiglu(gate.data(), up.data(), FD);
            cx::quantize_q8_avx2(xq, gate.data(), FD);
            gemv_wt_q8(ffn.data(), wd[l], xq, E, FD, pool.get(), vnni);
            for (int i = 0; i < E; i++) x[i] += ffn[i];
        }
        orc_rmsnorm(x.data(), x.data(), m->output_norm, E, m->rms_eps);
        cx::quantize_q8_avx2(xq, x.data(), E);
        gemv_wt_q8(logits.data(), head, xq, V, E, pool.get(), vnni);
        n_past++;
    }
    pool.reset();
    sched_setaffinity(0, sizeof(orig_aff), &orig_aff);
    return n;
}
