// capi_internal.hpp — shared between the C-ABI, the decoder and the kernels' launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/axf_hip.h"

struct axf_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    void* scratch = nullptr;  // grown on demand by eager entry points (never during capture)
    size_t scratch_bytes = 0;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    // benchmark helpers launch kernels directly instead of replaying a
    // captured graph (axf_hip_bench_set_eager; for runs under a profiler)
    int bench_eager = 0;
};

namespace axf {

constexpr int QK_K = 256;
constexpr int Q4K_BYTES = 144;
constexpr int Q6K_BYTES = 210;
constexpr int Q8_0_BYTES = 36;
constexpr int kMaxBlocksPerRow = 128;

int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* where);
int ctx_scratch(axf_ctx* ctx, size_t bytes, void** p);
// Argument checks shared by the GEMV/GEMM entry points (sizes, alignment of W,
// x and y; f32x: fp32 activation instead of Q8_0 blocks).
int check_gemv(const char* fn, int qtype, const void* W, const void* x, const float* y, int rows,
               int cols, size_t row_bytes, bool f32x);

enum class GemvKind { Q4K_Q8, Q4K_F32, Q6K_Q8, Q6K_F32 };

hipError_t launch_gemv(GemvKind kind, float* y, const void* W, const void* x, int rows, int nb,
                       long row_bytes, int accumulate, hipStream_t st);
// Q8_0-activation GEMV family with fused activation producers / consumers
// (kernels/gemv.hip, k_qgemv / k_qgemv2).
struct QGemvArgs {
    const uint8_t* W0;  // segment 0 weights, rows0 rows of rb0 bytes, output y0
    long rb0;
    int rows0;
    float* y0;
    const uint8_t* W1;  // segment 1 (two-type launch only)
    long rb1;
    int rows1;
    float* y1;
    int nwg0;           // workgroups of segment 0 (two-type launch; set by the launcher)
    int nb;             // 256-weight super-blocks per row (K / 256)
    int accumulate;     // y += v instead of y = v
    const uint8_t* xq8; // activation as Q8_0 blocks (QAct::Q8)
    const float* x;     // activation fp32 (QAct::Norm, QAct::F32)
    const float* nw;    // RMSNorm weight (QAct::Norm)
    float eps;
    int shape;          // launcher hint: kShapeNR1 or 0
    float* pv;          // launch_qgemv_argmax: per-workgroup maximum ...
    int* pi;            // ... and the first row index holding it
    // QAct::Norm with emb != nullptr: x is row `*tok_dev` (or `tok`) of the
    // Q4_K embedding matrix emb (emb_rb bytes per row), dequantised in the
    // prologue; workgroup 0 also writes it to x_out (no embedding kernel runs)
    const uint8_t* emb;
    long emb_rb;
    const int* tok_dev;
    int tok;
    float* x_out;
};
// kShapeNR1: one row per lane group (NR = 1) where the default places two,
// i.e. twice as many, smaller workgroups; the results are the same bits.
constexpr int kShapeNR1 = 1;
enum class QAct { Q8, Norm, F32 };
// One weight type (qtype 12 or 14).  swiglu: rows are blocks of R/2 gate rows
// then R/2 up rows (R = qgemv_rows_per_wg(nb, threads)); y0[i] = swiglu(gate_i, up_i).
hipError_t launch_qgemv(int qtype, QAct act, bool swiglu, QGemvArgs a, int threads,
                        hipStream_t st);
// QAct::Norm GEMV whose epilogue also writes each workgroup's (maximum, first
// row index) of y to a.pv / a.pi (the first stage of argmax); workgroups:
// qgemv_wgs(rows0, nb, threads, a.shape).  256 or 512 threads.
hipError_t launch_qgemv_argmax(int qtype, QGemvArgs a, int threads, hipStream_t st);
int qgemv_wgs(int rows, int nb, int threads, int shape);
// Q4_K segment (W0) and Q6_K segment (W1) over the same activation, one launch.
hipError_t launch_qgemv2(QAct act, QGemvArgs a, int threads, hipStream_t st);
int qgemv_threads(QAct act, int nb);  // default workgroup size for launch_qgemv
bool qgemv_threads_ok(QAct act, int nb, int threads);
int qgemv_rows_per_wg(int nb, int threads, int shape = 0);
// Q4_K / Q6_K x Q8_0 GEMM, Y token-major.  Auto: the dot4 kernel below
// kGemmMfmaMinT tokens, Stream up to kGemmStreamMaxT, Mfma above.  The
// matrix-core paths need gemm_scratch_bytes() of device scratch (activation
// re-layout, or Stream's split-K partials).  Stream: the Q4_K matrix-core
// kernel with the weights loaded straight into registers (T <= 64; it needs
// 16-byte-aligned W, XQ8 and row_bytes and otherwise runs as Mfma; Q6_K
// weights take Mfma).
enum class GemmPath { Auto = 0, Dot4 = 1, Mfma = 2, Stream = 3 };
constexpr int kGemmMfmaMinT = 8;
constexpr int kGemmStreamMaxT = 64;
GemmPath gemm_resolve(GemmPath path, int T);
size_t gemm_scratch_bytes(int qtype, GemmPath path, int T, int nb, int rows);
hipError_t launch_gemm_q4k_q8(float* Y, const void* W, const void* XQ8, int rows, int T, int nb,
                              long row_bytes, GemmPath path, void* scratch, hipStream_t st);
// Q6_K: the matrix-core kernel runs only when gemm_mfma_q6k_ok (the last
// row's last block ends on a 16-byte boundary, under 2 GiB from W); otherwise
// the dot4 kernel.
hipError_t launch_gemm_q6k_q8(float* Y, const void* W, const void* XQ8, int rows, int T, int nb,
                              long row_bytes, GemmPath path, void* scratch, hipStream_t st);
// the matrix-core kernels (kernels/gemm_mfma.hip)
size_t gemm_mfma_scratch_bytes(int T, int nb);
bool gemm_stream_q4k_ok(int T, int nb, int rows);
size_t gemm_stream_scratch_bytes(int T, int nb, int rows);
hipError_t launch_gemm_stream_q4k_q8(float* Y, const void* W, const void* XQ8, int rows, int T,
                                     int nb, long row_bytes, void* scratch, hipStream_t st);
// accumulate (Y +=): the fp16 kernel only (T >= 65); the int8 kernels below it refuse it
hipError_t launch_gemm_mfma_q4k_q8(float* Y, const void* W, const void* XQ8, int rows, int T,
                                   int nb, long row_bytes, void* scratch, hipStream_t st,
                                   int accumulate = 0);
size_t gemm_mfma_q6k_scratch_bytes(int T, int nb);
// The fp16 GEMMs on a re-layout written elsewhere (launch_rmsnorm_rows_prep):
// xh / dxt / gxt as k_gemm_prep16 lays them out for Tp tokens (a multiple of
// 64 serves both).  Q6_K: where gemm_f16_q6k_applies.  Q4_K with swiglu: the
// matrix is ffn_gate|ffn_up interleaved by blocks of 8 rows (rows % 128 ==
// 0); SwiGLU runs in the epilogue and h is written as the Q8_0 blocks of
// [T][rows/2] (hq8) and, when hf is set, as fp32 rows, instead of Y; with hxh
// set (Tp % 64 == 0) also their re-layout for the down projection (as
// launch_rmsnorm_rows_prep's, rows/64 blocks per token).
hipError_t launch_gemm_f16_q4k_xh(float* Y, uint8_t* hq8, float* hf, const void* W,
                                  const uint8_t* xh, const float* dxt, const float* gxt, int rows,
                                  int nb, long row_bytes, int T, int Tp, hipStream_t st,
                                  int accumulate, bool swiglu, uint8_t* hxh = nullptr,
                                  float* hdx2 = nullptr, float* hgx2 = nullptr,
                                  float* hdx4 = nullptr);
bool gemm_f16_q6k_applies(const void* W, int rows, int nb, long row_bytes, int T);
hipError_t launch_gemm_f16_q6k_xh(float* Y, const void* W, const uint8_t* xh, const float* dxt,
                                  int rows, int nb, long row_bytes, int T, int Tp, hipStream_t st,
                                  int accumulate);
bool gemm_mfma_q6k_ok(const void* W, int rows, int nb, long row_bytes);
hipError_t launch_gemm_mfma_q6k_q8(float* Y, const void* W, const void* XQ8, int rows, int T,
                                   int nb, long row_bytes, void* scratch, hipStream_t st,
                                   int accumulate = 0);
// Other weight types (kernels/gemv_misc.hip): nb = 32-element blocks per row.
// T tokens (T <= 65535): activation rows and y rows of token t follow each
// other (x + t*cols, xq8 + t*nb blocks, y + t*rows); accumulate adds to y.
hipError_t launch_gemv_q8w_q8(float* y, const void* W, const void* xq8, int rows, int nb,
                              long row_bytes, int accumulate, hipStream_t st, int T = 1);
hipError_t launch_gemv_q8w_f32(float* y, const void* W, const float* x, int rows, int nb,
                               long row_bytes, hipStream_t st, int accumulate = 0, int T = 1);
hipError_t launch_gemv_q5_0_f32(float* y, const void* W, const float* x, int rows, int nb,
                                long row_bytes, hipStream_t st, int accumulate = 0, int T = 1);
hipError_t launch_gemv_f16_f32(float* y, const void* W, const float* x, const float* bias,
                               int rows, int cols, hipStream_t st, int accumulate = 0, int T = 1);
// T fp32 token rows (Y token-major) through Q8_0 (8), Q5_0 (6) or F16 (1)
// weights (the batched prefill's gemm_wt_q8 fallback): from 16 tokens with
// scratch (gemm_misc_scratch_bytes; 16-byte aligned X) on the matrix cores,
// else each weight block dequantised once per 16 or 32 tokens on the VALU
hipError_t launch_gemm_misc_f32(int qtype, float* Y, const void* W, const float* X, int rows,
                                int cols, long row_bytes, int T, int accumulate, hipStream_t st,
                                float* scratch = nullptr, bool prepared = false);
size_t gemm_misc_scratch_bytes(int T, int cols);
// The matrix-core form runs (given scratch); its prepared activation rows in
// the scratch stay valid for further calls on the same X and cols (prepared =
// true) until the scratch is written otherwise.
bool gemm_misc_mfma_applies(int T, const float* X);
hipError_t launch_embed_misc(int qtype, float* out, const void* W, const int* tok_dev, int tok,
                             int T, int cols, long row_bytes, hipStream_t st);
// A decode stage of Q8_0 / Q5_0 / F16 matrices in one launch: RMSNorm(x) * nw
// in the prologue (the bits of launch_rmsnorm), then q, k, v rows (up to three
// matrices, y = W * activation) or, with swiglu, y = SwiGLU(gate, up) (mats[0]
// = gate with y = h, mats[1] = up).  n = K (n % 32 == 0, n <= 8192).
struct MiscMat {
    const void* W;
    long row_bytes;
    int rows;
    int qtype;
    float* y;
};
struct MiscStageArgs {
    const float* x;
    const float* nw;
    float eps;
    int n;
    const uint8_t* W[3];
    long rb[3];
    int rows[3];
    int qt[3];
    float* y[3];
    int nseg;
    int swiglu;
    int need_q8;
};
// False where the stage keeps the separate kernels: a K-quant matrix, K out of
// range, or rows whose types take different lanes per row.
bool misc_norm_stage_ok(const MiscMat* mats, int nmat, int n);
hipError_t launch_misc_norm_stage(const MiscMat* mats, int nmat, bool swiglu, const float* x,
                                  const float* nw, float eps, int n, hipStream_t st);
hipError_t launch_dequant_q4k(float* y, const void* W, long nblocks, hipStream_t st);
hipError_t launch_dequant_q6k(float* y, const void* W, long nblocks, hipStream_t st);
hipError_t launch_quantize_q8_0(void* y, const float* x, int n, hipStream_t st);
hipError_t launch_rmsnorm(float* y, void* yq8, const float* x, const float* w, int n, float eps,
                          hipStream_t st);
// rows independent RMSNorms of [rows][n] (same arithmetic as launch_rmsnorm)
// launch_rmsnorm_rows plus the fp16 GEMMs' re-layout of its Q8_0 blocks for Tp
// tokens (Tp % 64 == 0): xh (n/32 * Tp * 64 bytes), dx2 and gx2 (32-token
// groups), dx4 (64-token groups), n/32 * Tp floats each; rows T..Tp-1 zero
hipError_t launch_rmsnorm_rows_prep(float* y, void* yq8, const float* x, const float* w, int n,
                                    float eps, int T, int Tp, uint8_t* xh, float* dx2, float* gx2,
                                    float* dx4, hipStream_t st);
hipError_t launch_rmsnorm_rows(float* y, void* yq8, const float* x, const float* w, int n,
                               float eps, int rows, hipStream_t st);
hipError_t launch_rope_kv_rows(const float* k, int k_ld, const float* v, int v_ld,
                               const float* bk, const float* bv, float* kcache, float* vcache,
                               int pos0, int T, int n_kv_heads, int hd, const float* cos_t,
                               const float* sin_t, hipStream_t st);
hipError_t launch_swiglu_gu(void* outq8, const float* gu, int T, int n, int B, hipStream_t st,
                            float* out = nullptr);
hipError_t launch_embed_rows(int qtype, float* out, const void* W, const int* toks_dev, int T,
                             int nb, long row_bytes, hipStream_t st);
hipError_t launch_rope(float* dst, const float* src, const int* pos_dev, int pos, int n_heads,
                       int hd, const float* cos_t, const float* sin_t, hipStream_t st);
hipError_t launch_rope_qkv(float* q, const float* k, const float* v, float* kcache,
                           float* vcache, const int* pos_dev, int pos, int n_heads,
                           int n_kv_heads, int hd, const float* cos_t, const float* sin_t,
                           hipStream_t st);
// Single-token attention with RoPE and KV store fused (kernels/attention.hip).
struct AttnArgs {
    const float* q;      // [H*HD] query (raw projection; RoPE applied when cos_t != nullptr)
    const float* k;      // [KVH*HD] new key before bias and RoPE (used when store_kv)
    const float* v;      // [KVH*HD] new value before bias (used when store_kv)
    const float* bq;     // optional biases
    const float* bk;
    const float* bv;
    const float* cos_t;  // [n_ctx][HD/2] or nullptr (query already rotated)
    const float* sin_t;
    float* kcache;       // this layer, rows of KVH*HD floats
    float* vcache;
    const int* pos_dev;  // device position (graph replay) or nullptr
    int pos;             // current position: attention over rows 0..pos
    int n_heads, n_kv_heads, nsplit;
    int store_kv;        // write RoPE(k+bk) and v+bv to cache row pos
    float* part;         // [n_tok][H][nsplit][HD + 2]
    float* out;          // [H*HD] (row t at out + t*out_ld)
    uint8_t* outq8;      // Q8_0 blocks of out, or nullptr
    // Batched prefill: n_tok query rows (0 means 1), row t at q + t*q_ld, at
    // position pos + t, attending to cache rows 0..pos+t (store_kv must be 0).
    int n_tok, q_ld, out_ld;
    // prefill (k_attn_prefill_ks): when xh is set, also the out rows' Q8_0
    // blocks re-laid for the fp16 GEMMs for Tp tokens (as launch_rmsnorm_rows_prep)
    uint8_t* xh;
    float *dx2, *gx2, *dx4;
    int Tp;
};
int attn_nsplit(int max_seq);
hipError_t launch_attention_fused(const AttnArgs& a, int head_dim, hipStream_t st);
// Batched prefill attention on the matrix cores (n_tok query rows, K/V rows
// already in the cache; q, bq, cos_t/sin_t, kcache, vcache, pos, n_heads,
// n_kv_heads, out, outq8, n_tok, q_ld, out_ld are used).
hipError_t launch_attention_prefill(const AttnArgs& a, int head_dim, hipStream_t st);
// Per-head q/k RMSNorm models (order 1: before RoPE, 2: after): bias, norm and
// RoPE of the query rows in place and of the K rows into the cache, V rows
// (+ bias) into the cache, for n_tok rows at positions (pos_dev ? *pos_dev :
// pos) + t; the attention then runs with no bias, RoPE or store.
struct QkPrepArgs {
    float* q;
    int q_ld;
    const float *k, *v;
    int k_ld, v_ld;
    const float *bq, *bk, *bv;  // optional
    const float *qn, *kn;       // per-head norm weights (hd floats); nullptr: none
    int order;
    float eps;
    float *kcache, *vcache;
    const int* pos_dev;
    int pos;
    int n_heads, n_kv_heads, hd;
    const float *cos_t, *sin_t;
};
hipError_t launch_qk_prep(const QkPrepArgs& a, int n_tok, hipStream_t st);
hipError_t launch_swiglu(float* out, void* outq8, const float* gate, const float* up, int n,
                         hipStream_t st);
hipError_t launch_embed(int qtype, float* out, const void* W, const int* tok_dev, int tok,
                        int nb, long row_bytes, hipStream_t st);
int argmax_parts();
hipError_t launch_argmax(int* out, float* pv, int* pi, const float* x, int n, int* tokens,
                         int* step, int* pos, hipStream_t st);
// second stage alone: the nparts (value, index) pairs of a first stage
hipError_t launch_argmax_final(int* out, const float* pv, const int* pi, int nparts, int* tokens,
                               int* step, int* pos, hipStream_t st);
hipError_t launch_add(float* y, const float* a, const float* b, int n, hipStream_t st);
hipError_t launch_silu(float* y, const float* x, int n, hipStream_t st);
hipError_t launch_mul(float* y, const float* a, const float* b, int n, hipStream_t st);
hipError_t launch_set_int(int* p, int v, hipStream_t st);
// measurement kernel: read every 16-byte vector of [p, p + bytes) once
// (unroll 1/2/4/8 vectors in flight per thread, wgs workgroups of 256)
hipError_t launch_stream_read(const void* p, size_t bytes, int unroll, int wgs, uint32_t* sink,
                              hipStream_t st);
hipError_t launch_push_token(int* tokens, int* step, const int* tok, hipStream_t st);
// Device sampler (kernels/sample.hip).  sample_candidates returns the number of
// candidate keys (uint64) launch_sample needs in `cand`, 0 when k is beyond
// the device path.
int sample_candidates(int n_vocab, int k);
hipError_t launch_rep_penalty(float* logits, const int* hist, const int* hist_n, int last_n,
                              float penalty, int n_vocab, hipStream_t st);
hipError_t launch_sample(int* out, uint64_t* cand, const float* logits, int n_vocab,
                         float temperature, int top_k, float top_p, const float* r_table,
                         float r_fixed, int* tokens, int* step, int* pos, int* hist, int* hist_n,
                         hipStream_t st);
void sampling_uniforms(uint32_t seed, float* out, int n);
// effective k of sample() (llama_model.cpp:1473): 1 for greedy
inline int sample_k(const axf_sampling& s, int n_vocab) {
    if (!(s.temperature > 0.f)) return 1;
    return (s.top_k > 0 && s.top_k < n_vocab) ? s.top_k : n_vocab;
}

}  // namespace axf
