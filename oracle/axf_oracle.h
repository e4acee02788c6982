/*
 * axf_oracle.h — CPU parity oracle for the quantized decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * engine's x86 algorithm (songqiuyu/llm_core "AxonForge"), used as the checker
 * in tests/, in __graft_entry__.smoke() and as bench.py's cpu_baseline leg.
 * The product path (llm_core_amd/) never links, loads or calls it.
 *
 * Every function cites the reference file:line it follows.  Where the
 * reference uses explicit FMA intrinsics the restatement uses fmaf() at the
 * same place and keeps the reference's 8-lane accumulator layout and its
 * horizontal-sum order, so the GEMV restatements reproduce the compiled
 * reference kernels bit for bit (checked against oracle/_ref in tests/).
 * Built with -ffp-contract=off so that no other expression is fused.
 */
#ifndef AXF_ORACLE_H
#define AXF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML tensor type ids (reference include/axonforge/dtype.hpp:107-124). */
#define ORC_TYPE_F32 0
#define ORC_TYPE_Q4_K 12
#define ORC_TYPE_Q6_K 14

#define ORC_QK_K 256
#define ORC_Q4K_BYTES 144
#define ORC_Q6K_BYTES 210
#define ORC_Q8_0_BYTES 36

/* Q8_0 activation block: fp32 scale + 32 int8 (q8_block.hpp:8-15). */
typedef struct {
    float d;
    int8_t qs[32];
} orc_block_q8_0;

/* ---- scalar primitives -------------------------------------------------- */
float orc_fp16_to_fp32(uint16_t h);
void orc_get_scale_min_k4(int j, const uint8_t* scales, uint8_t* sc, uint8_t* m);

/* ---- dequantisation (bit-exact) ----------------------------------------- */
void orc_dequant_q4k(float* out, const uint8_t* blocks, int64_t nblocks);
void orc_dequant_q6k(float* out, const uint8_t* blocks, int64_t nblocks);

/* ---- F32-activation GEMV ------------------------------------------------- */
void orc_gemv_q4k_f32(float* y, const uint8_t* W, const float* x, int o_start, int o_end,
                      int in_dim, size_t row_bytes);
void orc_gemv_q6k_f32(float* y, const uint8_t* W, const float* x, int o_start, int o_end,
                      int in_dim, size_t row_bytes);

/* ---- Q8_0 activation path ----------------------------------------------- */
void orc_quantize_q8_0(orc_block_q8_0* y, const float* x, int k);
void orc_gemv_q4k_q8(float* y, const uint8_t* W, const orc_block_q8_0* xq8, int o_start,
                     int o_end, int in_dim, size_t row_bytes);
void orc_gemv_q6k_q8(float* y, const uint8_t* W, const orc_block_q8_0* xq8, int o_start,
                     int o_end, int in_dim, size_t row_bytes);
void orc_repack_q4k_r8(uint8_t* dst, const uint8_t* src, int nrows, int ncols);
void orc_gemm_q4k_q8(float* Y, const uint8_t* W, const orc_block_q8_0* XQ8, int M, int T,
                     int K, size_t row_bytes, int o_start, int o_end);

/* ---- decode-step operations ---------------------------------------------- */
void orc_rmsnorm(float* dst, const float* src, const float* w, int n, float eps);
void orc_rope_table(float* cos_t, float* sin_t, int head_dim, float theta, int max_pos);
void orc_rope(float* dst, const float* src, int pos, int n_heads, int head_dim,
              const float* cos_t, const float* sin_t);
float orc_dot_f32(const float* a, const float* b, int n);
void orc_softmax(float* x, int n);
void orc_attention(float* out, const float* q, const float* kcache, const float* vcache,
                   int seq, int n_heads, int n_kv_heads, int head_dim, float* scores);
float orc_exp_cephes(float x);
void orc_swiglu(float* gate, const float* up, int n);
int orc_argmax(const float* x, int n);
float orc_top2_margin(const float* x, int n);
void orc_gemv_q8_0w_q8(float* y, const uint8_t* W, const orc_block_q8_0* xq8, int o0, int o1,
                       int in, size_t rb);
void orc_gemv_q8_0w_f32(float* y, const uint8_t* W, const float* x, int o0, int o1, int in,
                        size_t rb);
void orc_gemv_q5_0_f32(float* y, const uint8_t* W, const float* x, int o0, int o1, int in,
                       size_t rb);
void orc_gemv_f16_f32(float* y, const uint16_t* W, const float* x, const float* bias, int o0,
                      int o1, int in);
void orc_dequant_row(float* out, int qtype, const uint8_t* row, int cols);
void orc_rep_penalty(float* logits, int n_vocab, const int32_t* hist, int n_hist, int last_n,
                     float penalty);
int orc_sample(const float* logits, int n_vocab, int top_k, float top_p, float temperature,
               float r, float* margin);

/* ---- decoder ------------------------------------------------------------- */
typedef struct {
    int type; /* ORC_TYPE_Q4_K or ORC_TYPE_Q6_K */
    const uint8_t* data;
} orc_wt;

typedef struct {
    const float* attn_norm;
    const float* ffn_norm;
    orc_wt wq, wk, wv, wo, wgate, wup, wdown;
    const float* bq; /* optional biases (Qwen2), may be NULL */
    const float* bk;
    const float* bv;
    const float* q_norm; /* optional per-head RMSNorm weights (head_dim floats), */
    const float* k_norm; /* used when orc_model.qk_norm_order != 0; may be NULL */
} orc_layer;

/* QkNormOrder (llama_model.cpp:955): 0 none, 1 before RoPE (qwen3), 2 after
 * RoPE (hunyuan-dense) */
enum { ORC_QK_NONE = 0, ORC_QK_BEFORE_ROPE = 1, ORC_QK_AFTER_ROPE = 2 };

typedef struct {
    int n_layer, n_embd, n_heads, n_kv_heads, ffn_dim, n_vocab, n_ctx;
    float rms_eps, rope_theta;
    orc_wt tok_embd;
    const float* output_norm;
    orc_wt output;
    const orc_layer* layers; /* n_layer entries */
    int qk_norm_order;       /* ORC_QK_* */
} orc_model;

typedef struct orc_state orc_state;

orc_state* orc_state_new(const orc_model* m);
void orc_state_free(orc_state* s);
float* orc_state_logits(orc_state* s);
float* orc_state_x(orc_state* s);
float* orc_state_kv_k(orc_state* s);
float* orc_state_kv_v(orc_state* s);
float* orc_state_q(orc_state* s);
float* orc_state_attn_out(orc_state* s);
float* orc_state_h(orc_state* s);
void orc_forward_token(const orc_model* m, orc_state* s, int token, int pos);
void orc_forward_layer(const orc_model* m, orc_state* s, int layer, int pos);
void orc_forward_batch(const orc_model* m, orc_state* s, const int32_t* tokens, int T,
                       int pos_start);
/* rms_norm_heads_inplace (llama_model.cpp:421-429): rms_norm_avx2 on each of
 * the n_heads head_dim-float heads of x with the one weight vector w; no-op
 * when w is NULL. */
void orc_rmsnorm_heads(float* x, const float* w, int n_heads, int head_dim, float eps);
int orc_generate_greedy(const orc_model* m, const int32_t* prompt, int n_prompt, int n_gen,
                        int batched_prefill, int32_t* out_tokens, float* out_margins);

#ifdef __cplusplus
}
#endif
#endif
