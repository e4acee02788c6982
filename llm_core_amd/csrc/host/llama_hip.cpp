// llama_hip.cpp — LLaMA-family decoder on one MI355X (the model-level `-b hip`
// hook, mirroring what llama_generate's backend branch selects at
// src/models/llama_model.cpp:1633-1642 and the per-token body of
// llama_forward_token, :1207-1333).
//
// Device layout (allocated once by axf_llama_load):
//   * weights in native GGUF blocks; attn_q|attn_k are placed back to back
//     when both are Q4_K (one GEMV whose output is q|k contiguous); ffn_gate
//     and ffn_up of one type are interleaved by row blocks (B gate rows, then
//     the same B up rows, B = half the rows of one GEMV workgroup), so one
//     GEMV workgroup holds both halves of its SwiGLU pairs;
//   * KV cache fp32 [layer][n_ctx][n_kv_heads*head_dim], K stored after RoPE
//     (LlamaState, :1102-1106);
//   * RoPE cos/sin table [n_ctx][head_dim/2] built on the host (:1031-1043);
//   * token id, position and step counters in device memory, so one captured
//     HIP graph replays every decode step: the argmax at the end of a step
//     writes the next token and advances the position.
//
// Step, per layer (six kernels):
//   1. q|k (Q4_K) and v (Q6_K) GEMVs in one launch, each workgroup computing
//      RMSNorm(x)*attn_norm -> Q8_0 in its prologue;
//   2./3. attention split (RoPE of q and k, store of k and v) and combine -> Q8_0;
//   4. o GEMV, x += o;
//   5. gate|up GEMV with RMSNorm(x)*ffn_norm -> Q8_0 prologue and SwiGLU
//      epilogue -> h (fp32);
//   6. down GEMV quantising h to Q8_0 in its prologue, x += down.
// Then the head GEMV with the final RMSNorm in its prologue, and argmax.
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../capi_internal.hpp"

using namespace axf;

namespace {

struct HostTensor {
    int qtype = -1;
    const void* host = nullptr;
    size_t bytes = 0;
};

struct DevW {
    int qtype = -1;
    uint8_t* d = nullptr;
    size_t row_bytes = 0;
};

struct Layer {
    float* attn_norm = nullptr;
    float* ffn_norm = nullptr;
    DevW wq, wk, wv, wo, wgate, wup, wdown;
    bool qk_fused = false;
    bool gu_interleaved = false;  // wgate holds gate and up rows interleaved by row blocks
    float *bq = nullptr, *bk = nullptr, *bv = nullptr;
    float *q_norm = nullptr, *k_norm = nullptr;  // per-head norms (qk_norm_order != 0)
};

}  // namespace

struct axf_llama {
    axf_ctx* ctx = nullptr;
    axf_llama_hparams hp{};
    int hd = 0, kv_embd = 0;
    std::map<std::string, HostTensor> pending;
    bool loaded = false;

    std::vector<void*> allocs;
    size_t dev_bytes = 0;

    DevW tok_embd, output;
    float* output_norm = nullptr;
    std::vector<Layer> layers;

    float *kv_k = nullptr, *kv_v = nullptr, *rope_cos = nullptr, *rope_sin = nullptr;
    float *x = nullptr, *qkv = nullptr, *attn_out = nullptr, *gateup = nullptr, *logits = nullptr;
    float* xb = nullptr;  // RMSNorm(x) * norm weight in fp32 (layers with Q5_0 / F16 matrices)
    float* h = nullptr;  // SwiGLU output, FD floats
    uint8_t* xq8 = nullptr;
    float* attn_part = nullptr;
    int nsplit = 0;
    float* arg_v = nullptr;  // argmax first-stage pairs: arg_n of each
    int* arg_i = nullptr;
    int arg_n = 0;
    int *d_token = nullptr, *d_pos = nullptr, *d_step = nullptr, *d_tokens = nullptr;
    int max_tokens = 0;

    // batched prefill buffers, allocated on first use for chunks of pf_cap tokens
    int pf_cap = 0;
    int* pf_tok = nullptr;
    float *pf_x = nullptr, *pf_qk = nullptr, *pf_v = nullptr, *pf_ao = nullptr, *pf_tmp = nullptr,
          *pf_gu = nullptr, *pf_part = nullptr;
    float *pf_xb = nullptr, *pf_h = nullptr;  // fp32 normalised rows and SwiGLU rows
    uint8_t *pf_q8 = nullptr, *pf_gemm = nullptr;
    // the fp16 GEMMs' re-layout of the RMSNorm rows (launch_rmsnorm_rows_prep)
    uint8_t* pf_xh = nullptr;
    float *pf_dx2 = nullptr, *pf_gx2 = nullptr, *pf_dx4 = nullptr;
    // and of h's Q8_0 blocks, written by the gate|up GEMM's SwiGLU epilogue
    uint8_t* pf_hxh = nullptr;
    float *pf_hdx2 = nullptr, *pf_hgx2 = nullptr, *pf_hdx4 = nullptr;
    // prefill attention: the matrix-core kernel, or (testing) the decode
    // split/combine kernels over a token grid
    bool pf_attn_split = false;

    // sampled generation (allocated on first use): penalty history (prompt and
    // generated tokens) and its length, the step's uniform draws, sort keys
    int *d_hist = nullptr, *d_hist_n = nullptr;
    float* d_r = nullptr;
    uint64_t* d_cand = nullptr;
    int cand_cap = 0;

    // graph[0]: greedy generation step (records the token, advances the position);
    // graph[1]: fixed-position step used to time decode at a given context;
    // graph[2]: sampled generation step, captured for the parameters in graph_smp
    hipGraph_t graph[3] = {nullptr, nullptr, nullptr};
    hipGraphExec_t exec[3] = {nullptr, nullptr, nullptr};
    axf_sampling graph_smp{};
};

namespace {

bool misc_type(int qtype) {
    return qtype == AXF_TYPE_Q8_0 || qtype == AXF_TYPE_Q5_0 || qtype == AXF_TYPE_F16;
}
bool kquant(int qtype) { return qtype == AXF_TYPE_Q4_K || qtype == AXF_TYPE_Q6_K; }

int dalloc(axf_llama* m, size_t bytes, void** p) {
    *p = nullptr;
    if (!bytes) return AXF_OK;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) return hip_fail(e, "axf_llama: hipMalloc");
    m->allocs.push_back(*p);
    m->dev_bytes += bytes;
    return AXF_OK;
}

#define LL_TRY(expr)              \
    do {                          \
        int rc_ = (expr);         \
        if (rc_) return rc_;      \
    } while (0)
#define LL_HIP(call)                                             \
    do {                                                         \
        hipError_t e_ = (call);                                  \
        if (e_ != hipSuccess) return hip_fail(e_, __func__);     \
    } while (0)

const HostTensor* find(axf_llama* m, const std::string& name) {
    auto it = m->pending.find(name);
    return it == m->pending.end() ? nullptr : &it->second;
}

int need(axf_llama* m, const std::string& name, const HostTensor** t) {
    *t = find(m, name);
    if (!*t) return fail(AXF_ERR_STATE, "axf_llama_load: missing tensor " + name);
    return AXF_OK;
}

int upload(axf_llama* m, void* dst, const void* src, size_t bytes) {
    LL_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, m->ctx->stream));
    LL_HIP(hipStreamSynchronize(m->ctx->stream));
    return AXF_OK;
}

int upload_f32(axf_llama* m, const std::string& name, int n, float** out, bool required) {
    const HostTensor* t = find(m, name);
    if (!t) {
        *out = nullptr;
        return required ? fail(AXF_ERR_STATE, "axf_llama_load: missing tensor " + name) : AXF_OK;
    }
    if (t->qtype != AXF_TYPE_F32 || t->bytes != (size_t)n * 4)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_load: " + name + " must be F32 of " +
                                             std::to_string(n) + " floats");
    void* p;
    LL_TRY(dalloc(m, t->bytes, &p));
    LL_TRY(upload(m, p, t->host, t->bytes));
    *out = static_cast<float*>(p);
    return AXF_OK;
}

// A layer matrix: Q4_K / Q6_K (rows of whole 256-weight super-blocks), or the
// types the reference's gemv_wt / gemv_wt_q8 also take (llama_model.cpp:670-831):
// Q8_0 and Q5_0 (32-weight blocks), F16 (rows of a multiple of 8 here: the
// kernel reads 16 bytes at a time).
int check_q(const std::string& name, const HostTensor* t, int rows, int cols) {
    if (kquant(t->qtype)) {
        if (cols % QK_K)
            return fail(AXF_ERR_UNSUPPORTED, "axf_llama_load: " + name +
                                                 " is Q4_K/Q6_K with rows that are not whole super-blocks");
    } else if (t->qtype == AXF_TYPE_Q8_0 || t->qtype == AXF_TYPE_Q5_0) {
        if (cols % 32)
            return fail(AXF_ERR_UNSUPPORTED, "axf_llama_load: " + name + " rows must be whole 32-blocks");
    } else if (t->qtype == AXF_TYPE_F16) {
        if (cols % 8)
            return fail(AXF_ERR_UNSUPPORTED, "axf_llama_load: " + name + " F16 rows must be a multiple of 8");
    } else {
        return fail(AXF_ERR_UNSUPPORTED,
                    "axf_llama_load: " + name + " must be Q4_K, Q6_K, Q8_0, Q5_0 or F16");
    }
    if (t->bytes != (size_t)rows * axf_row_bytes(t->qtype, cols))
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_load: " + name + " has wrong byte size");
    return AXF_OK;
}

// token_embd / output: also the other GGUF weight types of the reference's
// head and embedding paths (Q8_0, Q5_0, F16)
int upload_head(axf_llama* m, const std::string& name, int rows, int cols, DevW* w) {
    const HostTensor* t;
    LL_TRY(need(m, name, &t));
    LL_TRY(check_q(name, t, rows, cols));
    const size_t rb = axf_row_bytes(t->qtype, cols);
    void* p;
    LL_TRY(dalloc(m, t->bytes, &p));
    LL_TRY(upload(m, p, t->host, t->bytes));
    *w = DevW{t->qtype, static_cast<uint8_t*>(p), rb};
    return AXF_OK;
}

// Upload one or two quantized matrices; two matrices of the same qtype are
// placed back to back (so they can run as one GEMV).
int upload_pair(axf_llama* m, const std::string& n1, int rows1, const std::string& n2, int rows2,
                int cols, DevW* w1, DevW* w2, bool* fused) {
    const HostTensor *t1, *t2;
    LL_TRY(need(m, n1, &t1));
    LL_TRY(check_q(n1, t1, rows1, cols));
    if (w2) {
        LL_TRY(need(m, n2, &t2));
        LL_TRY(check_q(n2, t2, rows2, cols));
    }
    const bool pair = w2 && t2->qtype == t1->qtype && t1->qtype == AXF_TYPE_Q4_K;
    if (fused) *fused = pair;
    void* p;
    LL_TRY(dalloc(m, t1->bytes + (pair ? t2->bytes : 0), &p));
    LL_TRY(upload(m, p, t1->host, t1->bytes));
    *w1 = DevW{t1->qtype, static_cast<uint8_t*>(p), axf_row_bytes(t1->qtype, cols)};
    if (w2) {
        void* p2;
        if (pair) {
            p2 = static_cast<uint8_t*>(p) + t1->bytes;
        } else {
            LL_TRY(dalloc(m, t2->bytes, &p2));
        }
        LL_TRY(upload(m, p2, t2->host, t2->bytes));
        *w2 = DevW{t2->qtype, static_cast<uint8_t*>(p2), axf_row_bytes(t2->qtype, cols)};
    }
    return AXF_OK;
}

// workgroup size of the gate|up GEMV with the SwiGLU epilogue: 512 threads,
// twice the workgroups of 1024 (each repeats the RMSNorm prologue) but 8-wave
// instead of 16-wave workgroups to place (config-3 layer step 42.1 -> 41.3 us,
// 7B step 1.797 -> 1.794 ms, same box, alternating runs)
int gateup_threads(int) { return 512; }

// ffn_gate and ffn_up: of one qtype and with FD a multiple of the block B,
// uploaded as one matrix of row blocks [gate B rows][up B rows] ...; else
// separately.
int upload_gate_up(axf_llama* m, int l, Layer& L) {
    const auto& hp = m->hp;
    const int E = hp.n_embd, FD = hp.ffn_dim;
    const std::string b = "blk." + std::to_string(l) + ".";
    const HostTensor *tg, *tu;
    LL_TRY(need(m, b + "ffn_gate.weight", &tg));
    LL_TRY(check_q(b + "ffn_gate.weight", tg, FD, E));
    LL_TRY(need(m, b + "ffn_up.weight", &tu));
    LL_TRY(check_q(b + "ffn_up.weight", tu, FD, E));
    const int B = kquant(tg->qtype) ? qgemv_rows_per_wg(E / QK_K, gateup_threads(E)) / 2 : 1;
    L.gu_interleaved = kquant(tg->qtype) && tg->qtype == tu->qtype && FD % B == 0;
    if (!L.gu_interleaved) {
        LL_TRY(upload_pair(m, b + "ffn_gate.weight", FD, "", 0, E, &L.wgate, nullptr, nullptr));
        LL_TRY(upload_pair(m, b + "ffn_up.weight", FD, "", 0, E, &L.wup, nullptr, nullptr));
        return AXF_OK;
    }
    const size_t rb = axf_row_bytes(tg->qtype, E);
    std::vector<uint8_t> host(2 * (size_t)FD * rb);
    const auto* g = static_cast<const uint8_t*>(tg->host);
    const auto* u = static_cast<const uint8_t*>(tu->host);
    for (int j = 0; j < FD / B; j++) {
        std::memcpy(host.data() + (size_t)(2 * j) * B * rb, g + (size_t)j * B * rb, (size_t)B * rb);
        std::memcpy(host.data() + (size_t)(2 * j + 1) * B * rb, u + (size_t)j * B * rb,
                    (size_t)B * rb);
    }
    void* p;
    LL_TRY(dalloc(m, host.size(), &p));
    LL_TRY(upload(m, p, host.data(), host.size()));
    L.wgate = DevW{tg->qtype, static_cast<uint8_t*>(p), rb};
    L.wup = DevW{};
    return AXF_OK;
}

// Workgroup size of a decode GEMV (Q8_0 or normalised activation): the
// default, or, where the default leaves fewer than 256 workgroups (the
// 2048-wide layers of config 3, small heads), 256 threads with one row per
// lane group, 4-16x the workgroups (config-3 step 51.7 -> 49.2 us).
int decode_gemv_threads(QAct act, int rows, int nb, int* shape) {
    const int t = qgemv_threads(act, nb);
    const int rw = qgemv_rows_per_wg(nb, t);
    *shape = 0;
    if ((rows + rw - 1) / rw >= 256 || !qgemv_threads_ok(act, nb, 256)) return t;
    *shape = kShapeNR1;
    return 256;
}

QGemvArgs weights(const DevW& w, int rows, float* y, int cols) {
    QGemvArgs a{};
    a.W0 = w.d;
    a.rb0 = (long)w.row_bytes;
    a.rows0 = rows;
    a.y0 = y;
    a.nb = cols / QK_K;
    return a;
}

// y (+)= W * Q8_0(x) with x already Q8_0
hipError_t gemv_q8(const DevW& w, float* y, const void* xq8, int rows, int cols, bool acc,
                   hipStream_t st) {
    QGemvArgs a = weights(w, rows, y, cols);
    a.xq8 = static_cast<const uint8_t*>(xq8);
    a.accumulate = acc ? 1 : 0;
    const int threads = decode_gemv_threads(QAct::Q8, rows, a.nb, &a.shape);
    return launch_qgemv(w.qtype, QAct::Q8, false, a, threads, st);
}

// y (+)= W * activation by the reference's gemv_wt_q8 dispatch
// (llama_model.cpp:767-831): Q4_K, Q6_K and Q8_0 weights take the Q8_0
// activation xq8 (Q8_0: gemv_q8_0_weight_q8, :825-828), Q5_0 and F16 weights
// the fp32 activation xf through gemv_wt (:830).
hipError_t gemv_any(const DevW& w, float* y, const uint8_t* xq8, const float* xf, int rows,
                    int cols, bool acc, hipStream_t st) {
    if (kquant(w.qtype)) return gemv_q8(w, y, xq8, rows, cols, acc, st);
    if (w.qtype == AXF_TYPE_Q8_0)
        return launch_gemv_q8w_q8(y, w.d, xq8, rows, cols / 32, (long)w.row_bytes, acc ? 1 : 0, st);
    if (w.qtype == AXF_TYPE_Q5_0)
        return launch_gemv_q5_0_f32(y, w.d, xf, rows, cols / 32, (long)w.row_bytes, st, acc ? 1 : 0);
    return launch_gemv_f16_f32(y, w.d, xf, nullptr, rows, cols, st, acc ? 1 : 0);
}

// y = W * Q8_0(RMSNorm(x) * nw), the normalisation in the GEMV prologue;
// the SwiGLU variant (gate|up interleaved) runs 512-thread workgroups
hipError_t gemv_norm(const DevW& w, float* y, const float* x, const float* nw, float eps,
                     int rows, int cols, bool swiglu, hipStream_t st) {
    QGemvArgs a = weights(w, rows, y, cols);
    a.x = x;
    a.nw = nw;
    a.eps = eps;
    const int threads =
        swiglu ? gateup_threads(cols) : decode_gemv_threads(QAct::Norm, rows, a.nb, &a.shape);
    return launch_qgemv(w.qtype, QAct::Norm, swiglu, a, threads, st);
}

// logits = output * RMSNorm(x) * output_norm.  Q4_K / Q6_K heads fuse the norm
// into the GEMV prologue; the other types (gemv_wt_q8 / gemv_wt of the
// reference, llama_model.cpp:767-831) take the normalised row from k_rmsnorm:
// as Q8_0 activations for Q8_0 weights, fp32 for Q5_0 and F16.  `scratch`
// holds n_embd floats.
hipError_t head_logits(axf_llama* m, const float* x, float* scratch, hipStream_t st) {
    const auto& hp = m->hp;
    const DevW& w = m->output;
    if (!misc_type(w.qtype))
        return gemv_norm(w, m->logits, x, m->output_norm, hp.rms_eps, hp.n_vocab, hp.n_embd,
                         false, st);
    const bool q8 = w.qtype == AXF_TYPE_Q8_0;
    hipError_t e = launch_rmsnorm(scratch, q8 ? m->xq8 : nullptr, x, m->output_norm, hp.n_embd,
                                  hp.rms_eps, st);
    if (e != hipSuccess) return e;
    if (q8)
        return launch_gemv_q8w_q8(m->logits, w.d, m->xq8, hp.n_vocab, hp.n_embd / 32,
                                  (long)w.row_bytes, 0, st);
    if (w.qtype == AXF_TYPE_Q5_0)
        return launch_gemv_q5_0_f32(m->logits, w.d, scratch, hp.n_vocab, hp.n_embd / 32,
                                    (long)w.row_bytes, st);
    return launch_gemv_f16_f32(m->logits, w.d, scratch, nullptr, hp.n_vocab, hp.n_embd, st);
}

// The greedy head of a Q4_K / Q6_K output matrix (K <= 8192): logits and the
// first argmax stage in one launch (each workgroup's maximum and first index),
// then the final stage; *parts = the first stage's pairs.  False where the
// head takes head_logits + launch_argmax instead.
bool head_argmax_shape(const axf_llama* m, int* threads, int* shape, int* parts) {
    const auto& hp = m->hp;
    const int nb = hp.n_embd / QK_K;
    if (misc_type(m->output.qtype) || hp.n_embd % QK_K || !qgemv_threads_ok(QAct::Norm, nb, 512))
        return false;
    *threads = decode_gemv_threads(QAct::Norm, hp.n_vocab, nb, shape);
    *parts = qgemv_wgs(hp.n_vocab, nb, *threads, *shape);
    return true;
}

hipError_t head_argmax(axf_llama* m, bool record, bool advance_pos, hipStream_t st) {
    const auto& hp = m->hp;
    int threads, parts;
    QGemvArgs a = weights(m->output, hp.n_vocab, m->logits, hp.n_embd);
    if (!head_argmax_shape(m, &threads, &a.shape, &parts) || parts > m->arg_n)
        return hipErrorInvalidValue;
    a.x = m->x;
    a.nw = m->output_norm;
    a.eps = hp.rms_eps;
    a.pv = m->arg_v;
    a.pi = m->arg_i;
    hipError_t e = launch_qgemv_argmax(m->output.qtype, a, threads, st);
    if (e != hipSuccess) return e;
    return launch_argmax_final(m->d_token, m->arg_v, m->arg_i, parts, record ? m->d_tokens : nullptr,
                               record ? m->d_step : nullptr, advance_pos ? m->d_pos : nullptr, st);
}

// Embedding rows of T tokens (token ids on the device) or one token.
hipError_t embed(axf_llama* m, float* out, const int* tok_dev, int tok, int T, hipStream_t st) {
    const auto& hp = m->hp;
    const DevW& w = m->tok_embd;
    if (misc_type(w.qtype))
        return launch_embed_misc(w.qtype, out, w.d, tok_dev, tok, T, hp.n_embd, (long)w.row_bytes,
                                 st);
    if (T == 1 && (!tok_dev || tok_dev == m->d_token))
        return launch_embed(w.qtype, out, w.d, tok_dev, tok, hp.n_embd / QK_K, (long)w.row_bytes,
                            st);
    return launch_embed_rows(w.qtype, out, w.d, tok_dev, T, hp.n_embd / QK_K, (long)w.row_bytes, st);
}

// Enqueue one decoder layer; pos from device memory when pos_dev != nullptr.
// Stages first..last of the five (1: q|k|v projections, 2: attention, 3: o
// and x +=, 4: gate|up and SwiGLU, 5: down and x +=); the step runs 1..5.
constexpr int kDownThreads = 512;  // F32-prologue down projection workgroup

// Layer 0 of a step may take x from the embedding in its q|k|v prologue
// (Q4_K embeddings, fused q|k + v launch): embed_fusable, and the step then
// runs no embedding kernel.
bool embed_fusable(const axf_llama* m) {
    const Layer& L = m->layers[0];
    return m->tok_embd.qtype == AXF_TYPE_Q4_K && L.qk_fused && L.wv.qtype == AXF_TYPE_Q6_K;
}

// The q|k|v matrices of a layer as MiscMat segments (q|k as one matrix when
// fused); false unless every one is Q8_0 / Q5_0 / F16.
bool misc_qkv(const Layer& L, float* q, float* k, float* v, int qo, int kvo, MiscMat (&mm)[3]) {
    int n = 0;
    if (L.qk_fused) {
        mm[n++] = {L.wq.d, (long)L.wq.row_bytes, qo + kvo, L.wq.qtype, q};
    } else {
        mm[n++] = {L.wq.d, (long)L.wq.row_bytes, qo, L.wq.qtype, q};
        mm[n++] = {L.wk.d, (long)L.wk.row_bytes, kvo, L.wk.qtype, k};
    }
    mm[n++] = {L.wv.d, (long)L.wv.row_bytes, kvo, L.wv.qtype, v};
    for (int i = 0; i < n; i++)
        if (!misc_type(mm[i].qtype)) return false;
    return true;
}

hipError_t enqueue_layer(axf_llama* m, int l, const int* pos_dev, int pos, int first = 1,
                         int last = 5, const int* emb_tok_dev = nullptr, int emb_tok = -1) {
    const auto& hp = m->hp;
    const int E = hp.n_embd, H = hp.n_heads, KVH = hp.n_kv_heads, HD = m->hd, FD = hp.ffn_dim;
    const int qo = H * HD, kvo = KVH * HD;
    hipStream_t st = m->ctx->stream;
    const Layer& L = m->layers[l];
    float* q = m->qkv;
    float* k = m->qkv + qo;
    float* v = m->qkv + qo + kvo;
    const size_t loff = (size_t)l * hp.n_ctx * m->kv_embd;
    hipError_t e;
#define ST(call)               \
    if ((e = (call)) != hipSuccess) return e;
    auto stage = [&](int k) { return first <= k && k <= last; };
    // 1. q|k and v from RMSNorm(x) * attn_norm
    if (!stage(1)) {
    } else if (L.qk_fused && L.wv.qtype == AXF_TYPE_Q6_K) {
        QGemvArgs a = weights(L.wq, qo + kvo, q, E);
        a.W1 = L.wv.d;
        a.rb1 = (long)L.wv.row_bytes;
        a.rows1 = kvo;
        a.y1 = v;
        a.x = m->x;
        a.nw = L.attn_norm;
        a.eps = hp.rms_eps;
        if (emb_tok_dev || emb_tok >= 0) {  // x = the token's embedding row, written by the prologue
            a.emb = m->tok_embd.d;
            a.emb_rb = (long)m->tok_embd.row_bytes;
            a.tok_dev = emb_tok_dev;
            a.tok = emb_tok;
            a.x_out = m->x;
        }
        const int threads = decode_gemv_threads(QAct::Norm, a.rows0 + a.rows1, a.nb, &a.shape);
        ST(launch_qgemv2(QAct::Norm, a, threads, st));
    } else if (kquant(L.wq.qtype) && kquant(L.wk.qtype) && kquant(L.wv.qtype)) {
        if (L.qk_fused) {
            ST(gemv_norm(L.wq, q, m->x, L.attn_norm, hp.rms_eps, qo + kvo, E, false, st));
        } else {
            ST(gemv_norm(L.wq, q, m->x, L.attn_norm, hp.rms_eps, qo, E, false, st));
            ST(gemv_norm(L.wk, k, m->x, L.attn_norm, hp.rms_eps, kvo, E, false, st));
        }
        ST(gemv_norm(L.wv, v, m->x, L.attn_norm, hp.rms_eps, kvo, E, false, st));
    } else if (MiscMat mm[3]; misc_qkv(L, q, k, v, qo, kvo, mm) &&
                                misc_norm_stage_ok(mm, L.qk_fused ? 2 : 3, E)) {
        // all Q8_0 / Q5_0 / F16: the norm and the three projections in one launch
        ST(launch_misc_norm_stage(mm, L.qk_fused ? 2 : 3, false, m->x, L.attn_norm, hp.rms_eps, E,
                                  st));
    } else {
        // Q8_0 / Q5_0 / F16 projections: RMSNorm once (fp32 and Q8_0), then each
        // GEMV on the activation its type takes
        ST(launch_rmsnorm(m->xb, m->xq8, m->x, L.attn_norm, E, hp.rms_eps, st));
        if (L.qk_fused) {
            ST(gemv_any(L.wq, q, m->xq8, m->xb, qo + kvo, E, false, st));
        } else {
            ST(gemv_any(L.wq, q, m->xq8, m->xb, qo, E, false, st));
            ST(gemv_any(L.wk, k, m->xq8, m->xb, kvo, E, false, st));
        }
        ST(gemv_any(L.wv, v, m->xq8, m->xb, kvo, E, false, st));
    }
    // 2./3. attention -> Q8_0 of its output
    if (stage(2)) {
        const bool qkn = hp.qk_norm_order != 0;
        if (qkn) {  // per-head q/k norms: q, K, V finished and stored first
            QkPrepArgs pa{};
            pa.q = q;
            pa.q_ld = qo + 2 * kvo;
            pa.k = k;
            pa.v = v;
            pa.k_ld = pa.v_ld = qo + 2 * kvo;
            pa.bq = L.bq;
            pa.bk = L.bk;
            pa.bv = L.bv;
            pa.qn = L.q_norm;
            pa.kn = L.k_norm;
            pa.order = hp.qk_norm_order;
            pa.eps = hp.rms_eps;
            pa.kcache = m->kv_k + loff;
            pa.vcache = m->kv_v + loff;
            pa.pos_dev = pos_dev;
            pa.pos = pos;
            pa.n_heads = H;
            pa.n_kv_heads = KVH;
            pa.hd = HD;
            pa.cos_t = m->rope_cos;
            pa.sin_t = m->rope_sin;
            ST(launch_qk_prep(pa, 1, st));
        }
        AttnArgs a{};
        a.q = q;
        a.k = k;
        a.v = v;
        a.bq = qkn ? nullptr : L.bq;
        a.bk = L.bk;
        a.bv = L.bv;
        a.cos_t = qkn ? nullptr : m->rope_cos;
        a.sin_t = qkn ? nullptr : m->rope_sin;
        a.kcache = m->kv_k + loff;
        a.vcache = m->kv_v + loff;
        a.pos_dev = pos_dev;
        a.pos = pos;
        a.n_heads = H;
        a.n_kv_heads = KVH;
        a.nsplit = m->nsplit;
        a.store_kv = qkn ? 0 : 1;
        a.part = m->attn_part;
        a.out = m->attn_out;
        a.outq8 = m->xq8;
        ST(launch_attention_fused(a, HD, st));
    }
    // 4. x += o
    if (stage(3)) ST(gemv_any(L.wo, m->x, m->xq8, m->attn_out, E, qo, true, st));
    // 5. h = SwiGLU(gate, up) from RMSNorm(x) * ffn_norm
    if (!stage(4)) {
    } else if (L.gu_interleaved) {
        ST(gemv_norm(L.wgate, m->h, m->x, L.ffn_norm, hp.rms_eps, 2 * FD, E, true, st));
    } else if (kquant(L.wgate.qtype) && kquant(L.wup.qtype)) {
        ST(gemv_norm(L.wgate, m->gateup, m->x, L.ffn_norm, hp.rms_eps, FD, E, false, st));
        ST(gemv_norm(L.wup, m->gateup + FD, m->x, L.ffn_norm, hp.rms_eps, FD, E, false, st));
        ST(launch_swiglu(m->h, nullptr, m->gateup, m->gateup + FD, FD, st));
    } else if (MiscMat mm[2] = {{L.wgate.d, (long)L.wgate.row_bytes, FD, L.wgate.qtype, m->h},
                                {L.wup.d, (long)L.wup.row_bytes, FD, L.wup.qtype, nullptr}};
               misc_norm_stage_ok(mm, 2, E)) {
        // all Q8_0 / Q5_0 / F16: norm, gate, up and SwiGLU in one launch
        ST(launch_misc_norm_stage(mm, 2, true, m->x, L.ffn_norm, hp.rms_eps, E, st));
    } else {
        ST(launch_rmsnorm(m->xb, m->xq8, m->x, L.ffn_norm, E, hp.rms_eps, st));
        ST(gemv_any(L.wgate, m->gateup, m->xq8, m->xb, FD, E, false, st));
        ST(gemv_any(L.wup, m->gateup + FD, m->xq8, m->xb, FD, E, false, st));
        ST(launch_swiglu(m->h, nullptr, m->gateup, m->gateup + FD, FD, st));
    }
    // 6. x += down(Q8_0(h))
    if (stage(5) && !kquant(L.wdown.qtype)) {
        // Q8_0 weights take Q8_0(h), Q5_0 / F16 the fp32 h
        if (L.wdown.qtype == AXF_TYPE_Q8_0) ST(launch_quantize_q8_0(m->xq8, m->h, FD, st));
        ST(gemv_any(L.wdown, m->x, m->xq8, m->h, E, FD, true, st));
    } else if (stage(5)) {
        QGemvArgs a = weights(L.wdown, E, m->x, FD);
        a.x = m->h;
        a.accumulate = 1;
        // 512-thread workgroups where they apply: twice the workgroups of the
        // 1024-thread default (c3 down 2048 x 11008: 128 -> 256, measured
        // 55.2 -> 52.9 us per layer step; 7B: 1.910 -> 1.905 ms per step)
        const int thr = qgemv_threads_ok(QAct::F32, a.nb, kDownThreads) ? kDownThreads
                                                                         : qgemv_threads(QAct::F32, a.nb);
        ST(launch_qgemv(L.wdown.qtype, QAct::F32, false, a, thr, st));
    }
#undef ST
    return hipSuccess;
}

// Whole step: embedding of *d_token (or `token`), layers, final norm, head,
// argmax into d_token (+ tokens[step++] and pos++ when record != 0).
// The step's token choice: greedy argmax, or penalty + sampler (smp) with the
// draw r_table[*step] and the token appended to the penalty history.
hipError_t enqueue_pick(axf_llama* m, bool record, bool advance_pos, const axf_sampling* smp) {
    const auto& hp = m->hp;
    hipStream_t st = m->ctx->stream;
    if (!smp)
        return launch_argmax(m->d_token, m->arg_v, m->arg_i, m->logits, hp.n_vocab,
                             record ? m->d_tokens : nullptr, record ? m->d_step : nullptr,
                             advance_pos ? m->d_pos : nullptr, st);
    if (smp->rep_penalty != 1.0f) {
        hipError_t e = launch_rep_penalty(m->logits, m->d_hist, m->d_hist_n,
                                          smp->rep_penalty_last_n, smp->rep_penalty, hp.n_vocab, st);
        if (e != hipSuccess) return e;
    }
    return launch_sample(m->d_token, m->d_cand, m->logits, hp.n_vocab, smp->temperature,
                         smp->top_k, smp->top_p, m->d_r, 0.f, record ? m->d_tokens : nullptr,
                         record ? m->d_step : nullptr, advance_pos ? m->d_pos : nullptr,
                         m->d_hist, m->d_hist_n, st);
}

// The step's head: logits and the greedy pick (the fused argmax where it applies).
hipError_t head_pass(axf_llama* m, hipStream_t st) {
    int t, sh, parts;
    if (head_argmax_shape(m, &t, &sh, &parts)) return head_argmax(m, false, false, st);
    const hipError_t e = head_logits(m, m->x, m->attn_out, st);
    if (e != hipSuccess) return e;
    return enqueue_pick(m, false, false, nullptr);
}

hipError_t enqueue_step(axf_llama* m, bool device_state, int token, int pos, bool record,
                        const axf_sampling* smp = nullptr) {
    const auto& hp = m->hp;
    hipStream_t st = m->ctx->stream;
    const int* pd = device_state ? m->d_pos : nullptr;
    const int* td = device_state ? m->d_token : nullptr;
    hipError_t e = hipSuccess;
    const bool fuse = embed_fusable(m);
    if (!fuse && (e = embed(m, m->x, td, token, 1, st)) != hipSuccess) return e;
    for (int l = 0; l < hp.n_layer; l++) {
        const bool e0 = fuse && l == 0;
        e = enqueue_layer(m, l, pd, pos, 1, 5, e0 ? td : nullptr, e0 && !td ? token : -1);
        if (e != hipSuccess) return e;
    }
    int t, sh, parts;
    if (!smp && head_argmax_shape(m, &t, &sh, &parts))
        return head_argmax(m, record, device_state && record, st);
    if ((e = head_logits(m, m->x, m->attn_out, st)) != hipSuccess) return e;
    return enqueue_pick(m, record, device_state && record, smp);
}

// ---------------------------------------------------------------------------
// Batched prefill (llama_forward_batch, src/models/llama_model.cpp:1339-1462):
// per layer, for a chunk of T tokens at positions pos0 .. pos0+T-1,
//   RMSNorm rows -> Q8_0; q|k, v projections as T-token GEMMs (Q4_K on the
//   matrix cores, Q6_K with the dot4 kernel; the reference runs Q6_K per
//   token, gemm_wt_q8 :860-873); K (+bias, RoPE) and V (+bias) of every row
//   into the cache; causal attention of every row (q bias and RoPE inside);
//   o GEMM, x += o; RMSNorm rows -> Q8_0; gate|up GEMM, SwiGLU -> Q8_0;
//   down GEMM, x += down.
// Long prompts run as consecutive chunks; every row's arithmetic depends only
// on its own activations and the cache rows before it, so chunking does not
// change any result.  After the last chunk: the head of the last row.
// ---------------------------------------------------------------------------
int prefill_alloc(axf_llama* m) {
    if (m->pf_cap) return AXF_OK;
    const auto& hp = m->hp;
    const int E = hp.n_embd, FD = hp.ffn_dim, qo = hp.n_heads * m->hd, kvo = m->kv_embd;
    // chunk: up to 512 tokens (the matrix-core attention keeps no partials);
    // with the split/combine attention up to 256, its partials within 256 MiB
    const size_t part_per_tok = (size_t)hp.n_heads * m->nsplit * (m->hd + 2) * 4;
    int cap = m->pf_attn_split ? 256 : 512;
    while (m->pf_attn_split && cap > 16 && (size_t)cap * part_per_tok > ((size_t)256 << 20))
        cap /= 2;
    if (cap > hp.n_ctx) cap = hp.n_ctx;
    const size_t C = (size_t)cap;
    const int kmax = E > FD ? E : FD;
    void* p;
    LL_TRY(dalloc(m, C * 4, &p));
    m->pf_tok = static_cast<int*>(p);
    LL_TRY(dalloc(m, C * E * 4, &p));
    m->pf_x = static_cast<float*>(p);
    LL_TRY(dalloc(m, C * (qo + kvo) * 4, &p));
    m->pf_qk = static_cast<float*>(p);
    LL_TRY(dalloc(m, C * kvo * 4, &p));
    m->pf_v = static_cast<float*>(p);
    LL_TRY(dalloc(m, C * qo * 4, &p));
    m->pf_ao = static_cast<float*>(p);
    LL_TRY(dalloc(m, C * (E > qo ? E : qo) * 4, &p));
    m->pf_tmp = static_cast<float*>(p);
    LL_TRY(dalloc(m, C * 2 * FD * 4, &p));
    m->pf_gu = static_cast<float*>(p);
    LL_TRY(dalloc(m, C * E * 4, &p));
    m->pf_xb = static_cast<float*>(p);
    LL_TRY(dalloc(m, C * FD * 4, &p));
    m->pf_h = static_cast<float*>(p);
    if (m->pf_attn_split) {
        LL_TRY(dalloc(m, C * part_per_tok, &p));
        m->pf_part = static_cast<float*>(p);
    }
    LL_TRY(dalloc(m, C * (kmax > qo ? kmax : qo) / 32 * Q8_0_BYTES, &p));
    m->pf_q8 = static_cast<uint8_t*>(p);
    // GEMM scratch for every chunk size up to cap (the Auto path differs by T)
    int rmax = qo + kvo > 2 * FD ? qo + kvo : 2 * FD;
    if (E > rmax) rmax = E;
    size_t gs = 16;
    for (int t : {cap, 64, 16, 8})
        if (t <= cap)
            for (int qt : {AXF_TYPE_Q4_K, AXF_TYPE_Q6_K}) {
                const size_t b = gemm_scratch_bytes(qt, GemmPath::Auto, t, kmax / QK_K, rmax);
                if (b > gs) gs = b;
            }
    {  // the misc GEMM's hi/lo rows
        const size_t ms = gemm_misc_scratch_bytes(cap, kmax > qo ? kmax : qo);
        if (gs < ms) gs = ms;
    }
    LL_TRY(dalloc(m, gs, &p));
    m->pf_gemm = static_cast<uint8_t*>(p);
    {  // the RMSNorm rows' (and attention rows') fp16 re-layout, 64-token padding
        const size_t tp = (C + 63) / 64 * 64, nkb = (size_t)(E > qo ? E : qo) / 32;
        LL_TRY(dalloc(m, nkb * tp * 64, &p));
        m->pf_xh = static_cast<uint8_t*>(p);
        LL_TRY(dalloc(m, nkb * tp * 4 * 3, &p));
        m->pf_dx2 = static_cast<float*>(p);
        m->pf_gx2 = m->pf_dx2 + nkb * tp;
        m->pf_dx4 = m->pf_gx2 + nkb * tp;
        const size_t nkh = (size_t)FD / 32;
        LL_TRY(dalloc(m, nkh * tp * 64, &p));
        m->pf_hxh = static_cast<uint8_t*>(p);
        LL_TRY(dalloc(m, nkh * tp * 4 * 3, &p));
        m->pf_hdx2 = static_cast<float*>(p);
        m->pf_hgx2 = m->pf_hdx2 + nkh * tp;
        m->pf_hdx4 = m->pf_hgx2 + nkh * tp;
    }
    m->pf_cap = cap;
    return AXF_OK;
}

// Y[T][rows] = W * XQ8 rows (token-major), by weight type
hipError_t gemm_rows(axf_llama* m, const DevW& w, float* Y, const uint8_t* xq8, int rows, int T,
                     int cols, hipStream_t st) {
    if (w.qtype == AXF_TYPE_Q4_K)
        return launch_gemm_q4k_q8(Y, w.d, xq8, rows, T, cols / QK_K, (long)w.row_bytes,
                                  GemmPath::Auto, m->pf_gemm, st);
    return launch_gemm_q6k_q8(Y, w.d, xq8, rows, T, cols / QK_K, (long)w.row_bytes,
                              GemmPath::Auto, m->pf_gemm, st);
}

// Y[T][rows] += W x^T for the residual projections: the matrix-core kernels the
// automatic path picks for these sizes accumulate into Y themselves (the fp16
// Q4_K kernel from 65 tokens, the Q6_K kernel from 8); otherwise the product
// goes to tmp and a k_add follows.  Y + product is the same fp32 add either way.
hipError_t gemm_rows_add(axf_llama* m, const DevW& w, float* Y, const uint8_t* xq8, int rows,
                         int T, int cols, float* tmp, hipStream_t st) {
    const int nb = cols / QK_K;
    if (w.qtype == AXF_TYPE_Q4_K && T > kGemmStreamMaxT)
        return launch_gemm_mfma_q4k_q8(Y, w.d, xq8, rows, T, nb, (long)w.row_bytes, m->pf_gemm, st, 1);
    if (w.qtype == AXF_TYPE_Q6_K && T >= kGemmMfmaMinT && gemm_mfma_q6k_ok(w.d, rows, nb, (long)w.row_bytes))
        return launch_gemm_mfma_q6k_q8(Y, w.d, xq8, rows, T, nb, (long)w.row_bytes, m->pf_gemm, st, 1);
    hipError_t e = gemm_rows(m, w, tmp, xq8, rows, T, cols, st);
    if (e != hipSuccess) return e;
    return launch_add(Y, Y, tmp, T * rows, st);
}

// Y[T][rows] (+)= W rows by gemm_wt_q8's dispatch (llama_model.cpp:837-879):
// Q4_K and Q6_K on the Q8_0 rows; every other type, Q8_0 included (the batched
// path has no Q8_0 branch), on the fp32 rows XF through gemv_wt per token
// (:876-879).  xf_ready (optional): whether the GEMM scratch holds XF's
// prepared rows for the matrix-core misc GEMM, updated here; accumulate (misc
// types only) adds to Y.
hipError_t gemm_any(axf_llama* m, const DevW& w, float* Y, const uint8_t* xq8, const float* xf,
                    int rows, int T, int cols, hipStream_t st, bool* xf_ready = nullptr,
                    int accumulate = 0) {
    if (kquant(w.qtype)) {
        if (xf_ready) *xf_ready = false;  // the K-quant GEMMs use the scratch
        return gemm_rows(m, w, Y, xq8, rows, T, cols, st);
    }
    // from 8 tokens: each weight block dequantised once per 16 or 32 tokens, from
    // 16 on the matrix cores (XF's prepared rows in the GEMM scratch)
    if (T >= 8) {
        const hipError_t e = launch_gemm_misc_f32(w.qtype, Y, w.d, xf, rows, cols, (long)w.row_bytes,
                                                  T, accumulate, st,
                                                  reinterpret_cast<float*>(m->pf_gemm),
                                                  xf_ready && *xf_ready);
        if (xf_ready && gemm_misc_mfma_applies(T, xf)) *xf_ready = true;
        return e;
    }
    if (accumulate) return hipErrorInvalidValue;
    if (w.qtype == AXF_TYPE_Q8_0)
        return launch_gemv_q8w_f32(Y, w.d, xf, rows, cols / 32, (long)w.row_bytes, st, 0, T);
    if (w.qtype == AXF_TYPE_Q5_0)
        return launch_gemv_q5_0_f32(Y, w.d, xf, rows, cols / 32, (long)w.row_bytes, st, 0, T);
    return launch_gemv_f16_f32(Y, w.d, xf, nullptr, rows, cols, st, 0, T);
}

// x += W rows for a residual projection of another type: from 8 tokens the
// misc GEMM adds into x itself (the same fp32 add as k_add), below that the
// per-token GEMV writes pf_tmp and k_add follows.
hipError_t gemm_misc_add(axf_llama* m, const DevW& w, float* x, const uint8_t* xq8,
                         const float* xf, int rows, int T, int cols, hipStream_t st) {
    if (T >= 8) return gemm_any(m, w, x, xq8, xf, rows, T, cols, st, nullptr, 1);
    const hipError_t e = gemm_any(m, w, m->pf_tmp, xq8, xf, rows, T, cols, st);
    if (e != hipSuccess) return e;
    return launch_add(x, x, m->pf_tmp, T * rows, st);
}

hipError_t enqueue_prefill_layer(axf_llama* m, int l, int T, int pos0) {
    const auto& hp = m->hp;
    const int E = hp.n_embd, H = hp.n_heads, KVH = hp.n_kv_heads, HD = m->hd, FD = hp.ffn_dim;
    const int qo = H * HD, kvo = KVH * HD;
    hipStream_t st = m->ctx->stream;
    const Layer& L = m->layers[l];
    const size_t loff = (size_t)l * hp.n_ctx * m->kv_embd;
    hipError_t e;
#define ST(call)               \
    if ((e = (call)) != hipSuccess) return e;
    // q|k and v projections of RMSNorm(x) * attn_norm (fp32 rows too where a
    // projection of another type takes them)
    const bool f_qkv = !kquant(L.wq.qtype) || !kquant(L.wk.qtype) || !kquant(L.wv.qtype);
    // above 64 tokens the norm also writes the fp16 GEMMs' re-layout of its
    // Q8_0 blocks (k_gemm_prep16's, for 64-token groups), read by the Q4_K
    // q|k, v and gate|up GEMMs and the fp16 Q6_K v GEMM in place of their own
    const bool prep = T > kGemmStreamMaxT;
    const int Tp = (T + 63) / 64 * 64, nbE = E / QK_K;
    auto norm_rows = [&](const float* w, float* fp32_rows, bool re_layout) -> hipError_t {
        if (!re_layout)
            return launch_rmsnorm_rows(fp32_rows, m->pf_q8, m->pf_x, w, E, hp.rms_eps, T, st);
        return launch_rmsnorm_rows_prep(fp32_rows, m->pf_q8, m->pf_x, w, E, hp.rms_eps, T, Tp,
                                        m->pf_xh, m->pf_dx2, m->pf_gx2, m->pf_dx4, st);
    };
    // the re-layout only where a projection reads it
    auto reads_xh = [&](const DevW& w, int rows) {
        return w.qtype == AXF_TYPE_Q4_K ||
               (w.qtype == AXF_TYPE_Q6_K && gemm_f16_q6k_applies(w.d, rows, nbE, (long)w.row_bytes, T));
    };
    const bool qkv_xh = prep && (reads_xh(L.wq, L.qk_fused ? qo + kvo : qo) ||
                                 (!L.qk_fused && reads_xh(L.wk, kvo)) || reads_xh(L.wv, kvo));
    // Y = W rows of the normalised rows: the prepared fp16 GEMMs where they apply
    auto proj = [&](const DevW& w, float* Y, int rows, bool* xf_ready) -> hipError_t {
        if (!qkv_xh) return gemm_any(m, w, Y, m->pf_q8, m->pf_xb, rows, T, E, st, xf_ready);
        if (w.qtype == AXF_TYPE_Q4_K)
            return launch_gemm_f16_q4k_xh(Y, nullptr, nullptr, w.d, m->pf_xh, m->pf_dx2, m->pf_gx2,
                                          rows, nbE, (long)w.row_bytes, T, Tp, st, 0, false);
        if (w.qtype == AXF_TYPE_Q6_K && gemm_f16_q6k_applies(w.d, rows, nbE, (long)w.row_bytes, T))
            return launch_gemm_f16_q6k_xh(Y, w.d, m->pf_xh, m->pf_dx4, rows, nbE, (long)w.row_bytes,
                                          T, Tp, st, 0);
        return gemm_any(m, w, Y, m->pf_q8, m->pf_xb, rows, T, E, st, xf_ready);
    };
    ST(norm_rows(L.attn_norm, f_qkv ? m->pf_xb : nullptr, qkv_xh));
    bool xb_ready = false;  // the GEMM scratch holds pf_xb's prepared rows (misc types)
    float* q = m->pf_qk;
    float* k;
    int q_ld, k_ld;
    if (L.qk_fused) {
        ST(proj(L.wq, q, qo + kvo, &xb_ready));
        k = q + qo;
        q_ld = k_ld = qo + kvo;
    } else {
        k = q + (size_t)T * qo;
        q_ld = qo;
        k_ld = kvo;
        ST(proj(L.wq, q, qo, &xb_ready));
        ST(proj(L.wk, k, kvo, &xb_ready));
    }
    ST(proj(L.wv, m->pf_v, kvo, &xb_ready));
    // K, V rows into the cache, then attention of every row -> Q8_0
    const bool qkn = hp.qk_norm_order != 0;
    if (qkn) {  // per-head q/k norms: q rows finished in place, K/V rows stored
        QkPrepArgs pa{};
        pa.q = q;
        pa.q_ld = q_ld;
        pa.k = k;
        pa.k_ld = k_ld;
        pa.v = m->pf_v;
        pa.v_ld = kvo;
        pa.bq = L.bq;
        pa.bk = L.bk;
        pa.bv = L.bv;
        pa.qn = L.q_norm;
        pa.kn = L.k_norm;
        pa.order = hp.qk_norm_order;
        pa.eps = hp.rms_eps;
        pa.kcache = m->kv_k + loff;
        pa.vcache = m->kv_v + loff;
        pa.pos = pos0;
        pa.n_heads = H;
        pa.n_kv_heads = KVH;
        pa.hd = HD;
        pa.cos_t = m->rope_cos;
        pa.sin_t = m->rope_sin;
        ST(launch_qk_prep(pa, T, st));
    } else {
        ST(launch_rope_kv_rows(k, k_ld, m->pf_v, kvo, L.bk, L.bv, m->kv_k + loff,
                               m->kv_v + loff, pos0, T, KVH, HD, m->rope_cos, m->rope_sin, st));
    }
    // above 64 tokens the key-split attention (head dimension <= 128) also writes
    // the o projection's re-layout of its Q8_0 rows
    const bool o_prep = prep && !m->pf_attn_split && HD <= 128 && kquant(L.wo.qtype) &&
                        qo % QK_K == 0;
    {
        AttnArgs a{};
        a.q = q;
        a.bq = qkn ? nullptr : L.bq;
        a.cos_t = qkn ? nullptr : m->rope_cos;
        a.sin_t = qkn ? nullptr : m->rope_sin;
        a.kcache = m->kv_k + loff;
        a.vcache = m->kv_v + loff;
        a.pos = pos0;
        a.n_heads = H;
        a.n_kv_heads = KVH;
        a.nsplit = m->nsplit;
        a.store_kv = 0;
        a.part = m->pf_part;
        a.out = m->pf_ao;
        a.outq8 = m->pf_q8;
        a.n_tok = T;
        a.q_ld = q_ld;
        a.out_ld = qo;
        if (o_prep) {  // the o projection's re-layout (the q|k|v GEMMs are done with pf_xh)
            a.xh = m->pf_xh;
            a.dx2 = m->pf_dx2;
            a.gx2 = m->pf_gx2;
            a.dx4 = m->pf_dx4;
            a.Tp = Tp;
        }
        ST(m->pf_attn_split ? launch_attention_fused(a, HD, st)
                            : launch_attention_prefill(a, HD, st));
    }
    // x += o (the attention's fp32 rows pf_ao and their Q8_0 pf_q8)
    const int nbO = qo / QK_K;
    if (o_prep && L.wo.qtype == AXF_TYPE_Q4_K) {
        ST(launch_gemm_f16_q4k_xh(m->pf_x, nullptr, nullptr, L.wo.d, m->pf_xh, m->pf_dx2,
                                  m->pf_gx2, E, nbO, (long)L.wo.row_bytes, T, Tp, st, 1, false));
    } else if (o_prep && L.wo.qtype == AXF_TYPE_Q6_K &&
               gemm_f16_q6k_applies(L.wo.d, E, nbO, (long)L.wo.row_bytes, T)) {
        ST(launch_gemm_f16_q6k_xh(m->pf_x, L.wo.d, m->pf_xh, m->pf_dx4, E, nbO, (long)L.wo.row_bytes,
                                  T, Tp, st, 1));
    } else if (kquant(L.wo.qtype)) {
        ST(gemm_rows_add(m, L.wo, m->pf_x, m->pf_q8, E, T, qo, m->pf_tmp, st));
    } else {
        ST(gemm_misc_add(m, L.wo, m->pf_x, m->pf_q8, m->pf_ao, E, T, qo, st));
    }
    // SwiGLU(gate, up) of RMSNorm(x) * ffn_norm -> Q8_0 (and fp32 rows of h
    // where the down projection is of another type)
    const bool f_gu = !kquant(L.wgate.qtype) || !kquant(L.wup.qtype);
    const bool f_down = !kquant(L.wdown.qtype);
    const int B = L.gu_interleaved ? qgemv_rows_per_wg(E / QK_K, gateup_threads(E)) / 2 : 0;
    // SwiGLU in the fp16 gate|up GEMM's epilogue, on the norm's re-layout
    const bool sw = L.gu_interleaved && L.wgate.qtype == AXF_TYPE_Q4_K && B == 8 && prep &&
                    (2 * FD) % 128 == 0;
    const int nbF = FD / QK_K;
    // and h's re-layout from the epilogue where the down projection reads it
    const bool h_prep = sw && (L.wdown.qtype == AXF_TYPE_Q4_K ||
                               (L.wdown.qtype == AXF_TYPE_Q6_K &&
                                gemm_f16_q6k_applies(L.wdown.d, E, nbF, (long)L.wdown.row_bytes, T)));
    ST(norm_rows(L.ffn_norm, f_gu ? m->pf_xb : nullptr, sw));
    xb_ready = false;
    if (L.gu_interleaved) {
        if (sw) {
            // SwiGLU and its Q8_0 blocks in the fp16 GEMM's epilogue (the GEMM
            // reads its re-laid copy of the input blocks, so h may overwrite them)
            ST(launch_gemm_f16_q4k_xh(nullptr, m->pf_q8, f_down ? m->pf_h : nullptr, L.wgate.d,
                                      m->pf_xh, m->pf_dx2, m->pf_gx2, 2 * FD, nbE,
                                      (long)L.wgate.row_bytes, T, Tp, st, 0, true,
                                      h_prep ? m->pf_hxh : nullptr, m->pf_hdx2, m->pf_hgx2,
                                      m->pf_hdx4));
        } else {
            ST(gemm_rows(m, L.wgate, m->pf_gu, m->pf_q8, 2 * FD, T, E, st));
            ST(launch_swiglu_gu(m->pf_q8, m->pf_gu, T, FD, B, st, f_down ? m->pf_h : nullptr));
        }
    } else {
        ST(gemm_any(m, L.wgate, m->pf_gu, m->pf_q8, m->pf_xb, FD, T, E, st, &xb_ready));
        ST(gemm_any(m, L.wup, m->pf_gu + (size_t)T * FD, m->pf_q8, m->pf_xb, FD, T, E, st,
                    &xb_ready));
        ST(launch_swiglu(f_down ? m->pf_h : nullptr, m->pf_q8, m->pf_gu,
                         m->pf_gu + (size_t)T * FD, T * FD, st));
    }
    // x += down (on h's re-layout where the epilogue wrote it)
    if (h_prep && L.wdown.qtype == AXF_TYPE_Q4_K) {
        ST(launch_gemm_f16_q4k_xh(m->pf_x, nullptr, nullptr, L.wdown.d, m->pf_hxh, m->pf_hdx2,
                                  m->pf_hgx2, E, nbF, (long)L.wdown.row_bytes, T, Tp, st, 1, false));
    } else if (h_prep) {  // Q6_K where the fp16 kernel applies
        ST(launch_gemm_f16_q6k_xh(m->pf_x, L.wdown.d, m->pf_hxh, m->pf_hdx4, E, nbF,
                                  (long)L.wdown.row_bytes, T, Tp, st, 1));
    } else if (kquant(L.wdown.qtype)) {
        ST(gemm_rows_add(m, L.wdown, m->pf_x, m->pf_q8, E, T, FD, m->pf_tmp, st));
    } else {
        ST(gemm_misc_add(m, L.wdown, m->pf_x, m->pf_q8, m->pf_h, E, T, FD, st));
    }
#undef ST
    return hipSuccess;
}

// Tokens already on the device in pf_tok; logits of the last row when `head`.
int enqueue_prefill_chunk(axf_llama* m, int T, int pos0, bool head) {
    const auto& hp = m->hp;
    hipStream_t st = m->ctx->stream;
    LL_HIP(embed(m, m->pf_x, m->pf_tok, 0, T, st));
    for (int l = 0; l < hp.n_layer; l++) LL_HIP(enqueue_prefill_layer(m, l, T, pos0));
    if (head) {
        const float* xl = m->pf_x + (size_t)(T - 1) * hp.n_embd;
        LL_HIP(head_logits(m, xl, m->attn_out, st));
        // x = the last row after the final norm, as llama_forward_batch leaves s.x
        // (its in-place rms_norm_avx2 before the copy, :1452-1461)
        LL_HIP(launch_rmsnorm(m->x, nullptr, xl, m->output_norm, hp.n_embd, hp.rms_eps, st));
    }
    return AXF_OK;
}

int forward_batch(axf_llama* m, const int32_t* tokens, int T, int pos0) {
    LL_TRY(prefill_alloc(m));
    hipStream_t st = m->ctx->stream;
    for (int c0 = 0; c0 < T; c0 += m->pf_cap) {
        const int n = T - c0 < m->pf_cap ? T - c0 : m->pf_cap;
        LL_HIP(hipMemcpyAsync(m->pf_tok, tokens + c0, (size_t)n * 4, hipMemcpyHostToDevice, st));
        LL_TRY(enqueue_prefill_chunk(m, n, pos0 + c0, c0 + n == T));
        // the host token buffer of the next chunk reuses pf_tok
        LL_HIP(hipStreamSynchronize(st));
    }
    return AXF_OK;
}

// kind 0: generation step; kind 1: fixed-position step (no token record, no pos advance)
bool same_sampling(const axf_sampling& a, const axf_sampling& b) {
    return a.temperature == b.temperature && a.top_k == b.top_k && a.top_p == b.top_p &&
           a.rep_penalty == b.rep_penalty && a.rep_penalty_last_n == b.rep_penalty_last_n;
}

int ensure_graph(axf_llama* m, int kind, const axf_sampling* smp = nullptr) {
    if (kind == 2 && m->exec[2] && !same_sampling(m->graph_smp, *smp)) {
        LL_HIP(hipGraphExecDestroy(m->exec[2]));
        LL_HIP(hipGraphDestroy(m->graph[2]));
        m->exec[2] = nullptr;
        m->graph[2] = nullptr;
    }
    if (m->exec[kind]) return AXF_OK;
    hipStream_t st = m->ctx->stream;
    LL_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    hipError_t e = enqueue_step(m, true, 0, 0, kind != 1, kind == 2 ? smp : nullptr);
    hipGraph_t g = nullptr;
    hipError_t e2 = hipStreamEndCapture(st, &g);
    if (e != hipSuccess) return hip_fail(e, "axf_llama: capture");
    if (e2 != hipSuccess) return hip_fail(e2, "axf_llama: hipStreamEndCapture");
    m->graph[kind] = g;
    LL_HIP(hipGraphInstantiate(&m->exec[kind], g, nullptr, nullptr, 0));
    if (kind == 2) m->graph_smp = *smp;
    return AXF_OK;
}

int sampler_alloc(axf_llama* m, int n_cand) {
    void* p;
    if (!m->d_hist) {
        const size_t n = (size_t)m->hp.n_ctx + 2;
        LL_TRY(dalloc(m, n * 4, &p));
        m->d_hist = static_cast<int*>(p);
        LL_TRY(dalloc(m, 16, &p));
        m->d_hist_n = static_cast<int*>(p);
        LL_TRY(dalloc(m, n * 4, &p));
        m->d_r = static_cast<float*>(p);
    }
    if (n_cand > m->cand_cap) {
        // the sampled graph holds the old pointer: it is recaptured below
        LL_TRY(dalloc(m, (size_t)n_cand * 8, &p));
        m->d_cand = static_cast<uint64_t*>(p);
        m->cand_cap = n_cand;
        if (m->exec[2]) {
            LL_HIP(hipGraphExecDestroy(m->exec[2]));
            LL_HIP(hipGraphDestroy(m->graph[2]));
            m->exec[2] = nullptr;
            m->graph[2] = nullptr;
        }
    }
    return AXF_OK;
}

}  // namespace

extern "C" {

int axf_llama_create(axf_ctx* ctx, const axf_llama_hparams* hp, axf_llama** out) {
    if (!ctx || !hp || !out) return fail(AXF_ERR_INVALID_ARG, "axf_llama_create: null argument");
    *out = nullptr;
    const auto& h = *hp;
    if (h.n_layer <= 0 || h.n_embd <= 0 || h.n_heads <= 0 || h.n_kv_heads <= 0 ||
        h.ffn_dim <= 0 || h.n_vocab <= 0 || h.n_ctx <= 0)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_create: non-positive hyperparameter");
    if (h.n_embd % h.n_heads || h.n_heads % h.n_kv_heads)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_create: heads do not divide");
    const int hd = h.n_embd / h.n_heads;
    if (h.n_heads / h.n_kv_heads > 8)
        return fail(AXF_ERR_UNSUPPORTED, "axf_llama_create: more than 8 query heads per kv head");
    if (h.n_ctx > 32768)
        return fail(AXF_ERR_UNSUPPORTED, "axf_llama_create: n_ctx above 32768");
    if (hd != 64 && hd != 128 && hd != 256)
        return fail(AXF_ERR_UNSUPPORTED, "axf_llama_create: head_dim must be 64, 128 or 256");
    // Q8_0 activation blocks of 32; matrices of whole super-blocks (Q4_K / Q6_K)
    // are checked per tensor at load
    if (h.n_embd % 32 || h.ffn_dim % 32)
        return fail(AXF_ERR_UNSUPPORTED, "axf_llama_create: n_embd and ffn_dim must be multiples of 32");
    if (h.n_embd > kMaxBlocksPerRow * QK_K || h.ffn_dim > kMaxBlocksPerRow * QK_K)
        return fail(AXF_ERR_UNSUPPORTED, "axf_llama_create: dimension above 32768");
    if (h.n_embd > 8192)  // the GEMVs that fuse RMSNorm take K <= 8192
        return fail(AXF_ERR_UNSUPPORTED, "axf_llama_create: n_embd above 8192");
    if (h.qk_norm_order < 0 || h.qk_norm_order > 2)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_create: qk_norm_order must be 0, 1 or 2");
    auto* m = new axf_llama();
    m->ctx = ctx;
    m->hp = h;
    m->hd = hd;
    m->kv_embd = h.n_kv_heads * hd;
    *out = m;
    return AXF_OK;
}

int axf_llama_destroy(axf_llama* m) {
    if (!m) return AXF_OK;
    (void)hipStreamSynchronize(m->ctx->stream);
    for (int k = 0; k < 3; k++) {
        if (m->exec[k]) (void)hipGraphExecDestroy(m->exec[k]);
        if (m->graph[k]) (void)hipGraphDestroy(m->graph[k]);
    }
    for (void* p : m->allocs) (void)hipFree(p);
    delete m;
    return AXF_OK;
}

int axf_llama_set_tensor(axf_llama* m, const char* name, int qtype, const void* host,
                         size_t bytes) {
    if (!m || !name || !host) return fail(AXF_ERR_INVALID_ARG, "axf_llama_set_tensor: null argument");
    if (m->loaded) return fail(AXF_ERR_STATE, "axf_llama_set_tensor: model already loaded");
    m->pending[name] = HostTensor{qtype, host, bytes};
    return AXF_OK;
}

int axf_llama_load(axf_llama* m) {
    if (!m) return fail(AXF_ERR_INVALID_ARG, "axf_llama_load: null model");
    if (m->loaded) return AXF_OK;
    LL_HIP(hipSetDevice(m->ctx->device));
    const auto& hp = m->hp;
    const int E = hp.n_embd, FD = hp.ffn_dim, qo = hp.n_heads * m->hd, kvo = m->kv_embd;
    char nm[128];
    {
        LL_TRY(upload_head(m, "token_embd.weight", hp.n_vocab, E, &m->tok_embd));
        // output.weight falls back to token_embd (make_wt_opt, llama_model.cpp:660-667)
        if (find(m, "output.weight"))
            LL_TRY(upload_head(m, "output.weight", hp.n_vocab, E, &m->output));
        else
            m->output = m->tok_embd;
        LL_TRY(upload_f32(m, "output_norm.weight", E, &m->output_norm, true));
    }
    m->layers.resize(hp.n_layer);
    for (int l = 0; l < hp.n_layer; l++) {
        Layer& L = m->layers[l];
        auto n = [&](const char* s) {
            std::snprintf(nm, sizeof(nm), "blk.%d.%s", l, s);
            return std::string(nm);
        };
        LL_TRY(upload_f32(m, n("attn_norm.weight"), E, &L.attn_norm, true));
        LL_TRY(upload_f32(m, n("ffn_norm.weight"), E, &L.ffn_norm, true));
        LL_TRY(upload_pair(m, n("attn_q.weight"), qo, n("attn_k.weight"), kvo, E, &L.wq, &L.wk,
                           &L.qk_fused));
        LL_TRY(upload_pair(m, n("attn_v.weight"), kvo, "", 0, E, &L.wv, nullptr, nullptr));
        LL_TRY(upload_pair(m, n("attn_output.weight"), E, "", 0, qo, &L.wo, nullptr, nullptr));
        LL_TRY(upload_gate_up(m, l, L));
        LL_TRY(upload_pair(m, n("ffn_down.weight"), E, "", 0, FD, &L.wdown, nullptr, nullptr));
        LL_TRY(upload_f32(m, n("attn_q.bias"), qo, &L.bq, false));
        LL_TRY(upload_f32(m, n("attn_k.bias"), kvo, &L.bk, false));
        LL_TRY(upload_f32(m, n("attn_v.bias"), kvo, &L.bv, false));
        if (hp.qk_norm_order) {  // the reference ignores them without an order
            LL_TRY(upload_f32(m, n("attn_q_norm.weight"), m->hd, &L.q_norm, false));
            LL_TRY(upload_f32(m, n("attn_k_norm.weight"), m->hd, &L.k_norm, false));
        }
    }
    // KV cache and buffers
    const size_t kv_floats = (size_t)hp.n_layer * hp.n_ctx * m->kv_embd;
    void* p;
    LL_TRY(dalloc(m, kv_floats * 4, &p));
    m->kv_k = static_cast<float*>(p);
    LL_TRY(dalloc(m, kv_floats * 4, &p));
    m->kv_v = static_cast<float*>(p);
    LL_HIP(hipMemsetAsync(m->kv_k, 0, kv_floats * 4, m->ctx->stream));
    LL_HIP(hipMemsetAsync(m->kv_v, 0, kv_floats * 4, m->ctx->stream));
    {
        std::vector<float> c((size_t)hp.n_ctx * m->hd / 2), s(c.size());
        axf_rope_table(c.data(), s.data(), m->hd, hp.rope_theta, hp.n_ctx);
        LL_TRY(dalloc(m, c.size() * 4, &p));
        m->rope_cos = static_cast<float*>(p);
        LL_TRY(upload(m, p, c.data(), c.size() * 4));
        LL_TRY(dalloc(m, s.size() * 4, &p));
        m->rope_sin = static_cast<float*>(p);
        LL_TRY(upload(m, p, s.data(), s.size() * 4));
    }
    LL_TRY(dalloc(m, (size_t)E * 4, &p));
    m->x = static_cast<float*>(p);
    LL_TRY(dalloc(m, (size_t)E * 4, &p));
    m->xb = static_cast<float*>(p);
    LL_TRY(dalloc(m, (size_t)(qo + 2 * kvo) * 4, &p));
    m->qkv = static_cast<float*>(p);
    LL_TRY(dalloc(m, (size_t)qo * 4, &p));
    m->attn_out = static_cast<float*>(p);
    LL_TRY(dalloc(m, (size_t)2 * FD * 4, &p));
    m->gateup = static_cast<float*>(p);
    LL_TRY(dalloc(m, (size_t)FD * 4, &p));
    m->h = static_cast<float*>(p);
    LL_TRY(dalloc(m, (size_t)hp.n_vocab * 4, &p));
    m->logits = static_cast<float*>(p);
    LL_TRY(dalloc(m, (size_t)((E > FD ? E : FD) / 32) * Q8_0_BYTES, &p));
    m->xq8 = static_cast<uint8_t*>(p);
    m->nsplit = attn_nsplit(hp.n_ctx);
    LL_TRY(dalloc(m, (size_t)hp.n_heads * m->nsplit * (m->hd + 2) * 4, &p));
    m->attn_part = static_cast<float*>(p);
    {
        int t, sh, parts = 0;
        m->arg_n = argmax_parts();
        if (head_argmax_shape(m, &t, &sh, &parts) && parts > m->arg_n) m->arg_n = parts;
    }
    LL_TRY(dalloc(m, (size_t)m->arg_n * 8, &p));
    m->arg_v = static_cast<float*>(p);
    m->arg_i = reinterpret_cast<int*>(m->arg_v + m->arg_n);
    m->max_tokens = hp.n_ctx + 1;
    LL_TRY(dalloc(m, (size_t)(3 + m->max_tokens) * 4, &p));
    m->d_token = static_cast<int*>(p);
    m->d_pos = m->d_token + 1;
    m->d_step = m->d_token + 2;
    m->d_tokens = m->d_token + 3;
    LL_HIP(hipMemsetAsync(m->d_token, 0, (size_t)(3 + m->max_tokens) * 4, m->ctx->stream));
    LL_HIP(hipStreamSynchronize(m->ctx->stream));
    m->pending.clear();
    m->loaded = true;
    return AXF_OK;
}

size_t axf_llama_device_bytes(axf_llama* m) { return m ? m->dev_bytes : 0; }

int axf_llama_get_hparams(const axf_llama* m, axf_llama_hparams* hp) {
    if (!m || !hp) return fail(AXF_ERR_INVALID_ARG, "axf_llama_get_hparams: null argument");
    *hp = m->hp;
    return AXF_OK;
}

#define LL_LOADED(m)                                                                       \
    if (!(m)) return fail(AXF_ERR_INVALID_ARG, std::string(__func__) + ": null model");     \
    if (!(m)->loaded) return fail(AXF_ERR_STATE, std::string(__func__) + ": model not loaded")

int axf_llama_set_x(axf_llama* m, const float* x) {
    LL_LOADED(m);
    return upload(m, m->x, x, (size_t)m->hp.n_embd * 4);
}

int axf_llama_get_x(axf_llama* m, float* x) {
    LL_LOADED(m);
    LL_HIP(hipMemcpyAsync(x, m->x, (size_t)m->hp.n_embd * 4, hipMemcpyDeviceToHost,
                          m->ctx->stream));
    LL_HIP(hipStreamSynchronize(m->ctx->stream));
    return AXF_OK;
}

int axf_llama_set_kv(axf_llama* m, int layer, const float* k, const float* v, int n_pos) {
    LL_LOADED(m);
    if (layer < 0 || layer >= m->hp.n_layer || n_pos < 0 || n_pos > m->hp.n_ctx || !k || !v)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_set_kv: bad arguments");
    const size_t off = (size_t)layer * m->hp.n_ctx * m->kv_embd;
    const size_t bytes = (size_t)n_pos * m->kv_embd * 4;
    LL_TRY(upload(m, m->kv_k + off, k, bytes));
    LL_TRY(upload(m, m->kv_v + off, v, bytes));
    return AXF_OK;
}

int axf_llama_fill_kv_random(axf_llama* m, int n_pos, uint64_t seed) {
    LL_LOADED(m);
    if (n_pos < 0 || n_pos > m->hp.n_ctx)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_fill_kv_random: bad n_pos");
    std::vector<float> buf((size_t)n_pos * m->kv_embd);
    for (int l = 0; l < m->hp.n_layer; l++) {
        const size_t off = (size_t)l * m->hp.n_ctx * m->kv_embd;
        LL_TRY(axf_synth_normal(buf.data(), (int64_t)buf.size(), seed + 2 * l, 0.f, 1.f));
        LL_TRY(upload(m, m->kv_k + off, buf.data(), buf.size() * 4));
        LL_TRY(axf_synth_normal(buf.data(), (int64_t)buf.size(), seed + 2 * l + 1, 0.f, 1.f));
        LL_TRY(upload(m, m->kv_v + off, buf.data(), buf.size() * 4));
    }
    return AXF_OK;
}

int axf_llama_get_logits(axf_llama* m, float* logits) {
    LL_LOADED(m);
    LL_HIP(hipMemcpyAsync(logits, m->logits, (size_t)m->hp.n_vocab * 4, hipMemcpyDeviceToHost,
                          m->ctx->stream));
    LL_HIP(hipStreamSynchronize(m->ctx->stream));
    return AXF_OK;
}

int axf_llama_forward_layer(axf_llama* m, int layer, int pos) {
    LL_LOADED(m);
    if (layer < 0 || layer >= m->hp.n_layer || pos < 0 || pos >= m->hp.n_ctx)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_forward_layer: bad layer/pos");
    LL_HIP(enqueue_layer(m, layer, nullptr, pos));
    LL_HIP(hipStreamSynchronize(m->ctx->stream));
    return AXF_OK;
}

int axf_llama_forward_layer_stages(axf_llama* m, int layer, int pos, int first, int last) {
    LL_LOADED(m);
    if (layer < 0 || layer >= m->hp.n_layer || pos < 0 || pos >= m->hp.n_ctx || first < 1 ||
        last > 5 || first > last)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_forward_layer_stages: bad layer/pos/stages");
    LL_HIP(enqueue_layer(m, layer, nullptr, pos, first, last));
    LL_HIP(hipStreamSynchronize(m->ctx->stream));
    return AXF_OK;
}

int axf_llama_get_buffer(axf_llama* m, int which, void* out, size_t bytes) {
    LL_LOADED(m);
    const auto& hp = m->hp;
    const size_t qo = (size_t)hp.n_heads * m->hd, kvo = (size_t)m->kv_embd;
    const void* src = nullptr;
    size_t n = 0;
    switch (which) {
        case AXF_LLAMA_BUF_X: src = m->x; n = (size_t)hp.n_embd * 4; break;
        case AXF_LLAMA_BUF_QKV: src = m->qkv; n = (qo + 2 * kvo) * 4; break;
        case AXF_LLAMA_BUF_ATTN: src = m->attn_out; n = qo * 4; break;
        case AXF_LLAMA_BUF_ATTN_Q8: src = m->xq8; n = qo / 32 * Q8_0_BYTES; break;
        case AXF_LLAMA_BUF_H: src = m->h; n = (size_t)hp.ffn_dim * 4; break;
        case AXF_LLAMA_BUF_LOGITS: src = m->logits; n = (size_t)hp.n_vocab * 4; break;
        default: return fail(AXF_ERR_INVALID_ARG, "axf_llama_get_buffer: unknown buffer");
    }
    if (!out || bytes != n)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_get_buffer: wrong size (want " +
                                             std::to_string(n) + " bytes)");
    LL_HIP(hipMemcpyAsync(out, src, n, hipMemcpyDeviceToHost, m->ctx->stream));
    LL_HIP(hipStreamSynchronize(m->ctx->stream));
    return AXF_OK;
}

int axf_llama_get_kv(axf_llama* m, int layer, float* k, float* v, int pos0, int n_pos) {
    LL_LOADED(m);
    if (layer < 0 || layer >= m->hp.n_layer || pos0 < 0 || n_pos < 0 ||
        pos0 + n_pos > m->hp.n_ctx || (n_pos && (!k || !v)))
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_get_kv: bad arguments");
    const size_t off = ((size_t)layer * m->hp.n_ctx + pos0) * m->kv_embd;
    const size_t bytes = (size_t)n_pos * m->kv_embd * 4;
    LL_HIP(hipMemcpyAsync(k, m->kv_k + off, bytes, hipMemcpyDeviceToHost, m->ctx->stream));
    LL_HIP(hipMemcpyAsync(v, m->kv_v + off, bytes, hipMemcpyDeviceToHost, m->ctx->stream));
    LL_HIP(hipStreamSynchronize(m->ctx->stream));
    return AXF_OK;
}

int axf_llama_forward_token(axf_llama* m, int token, int pos) {
    LL_LOADED(m);
    if (token < 0 || token >= m->hp.n_vocab || pos < 0 || pos >= m->hp.n_ctx)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_forward_token: bad token/pos");
    LL_HIP(enqueue_step(m, false, token, pos, false));
    LL_HIP(hipStreamSynchronize(m->ctx->stream));
    return AXF_OK;
}

int axf_llama_forward_batch(axf_llama* m, const int32_t* tokens, int T, int pos_start) {
    LL_LOADED(m);
    if (!tokens || T <= 0 || pos_start < 0 || pos_start + T > m->hp.n_ctx)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_forward_batch: bad tokens/positions");
    for (int i = 0; i < T; i++)
        if (tokens[i] < 0 || tokens[i] >= m->hp.n_vocab)
            return fail(AXF_ERR_INVALID_ARG, "axf_llama_forward_batch: token out of range");
    LL_TRY(forward_batch(m, tokens, T, pos_start));
    LL_HIP(hipStreamSynchronize(m->ctx->stream));
    return AXF_OK;
}

int axf_llama_bench_prefill(axf_llama* m, int T, int reps, float* ms) {
    LL_LOADED(m);
    if (!ms || T <= 0 || T > m->hp.n_ctx || reps <= 0)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_bench_prefill: bad arguments");
    std::vector<int32_t> toks(T);
    for (int i = 0; i < T; i++) toks[i] = (int32_t)((1 + 7 * (int64_t)i) % m->hp.n_vocab);
    LL_TRY(forward_batch(m, toks.data(), T, 0));  // warm-up (allocations, code)
    float total = 0.f;
    for (int r = 0; r < reps; r++) {
        LL_HIP(hipEventRecord(m->ctx->ev0, m->ctx->stream));
        LL_TRY(forward_batch(m, toks.data(), T, 0));
        LL_HIP(hipEventRecord(m->ctx->ev1, m->ctx->stream));
        LL_HIP(hipEventSynchronize(m->ctx->ev1));
        float t = 0.f;
        LL_HIP(hipEventElapsedTime(&t, m->ctx->ev0, m->ctx->ev1));
        total += t;
    }
    *ms = total / (float)reps;
    return AXF_OK;
}

int axf_llama_generate(axf_llama* m, const int32_t* prompt, int n_prompt, int n_gen,
                       int32_t* out_tokens, int use_graph) {
    return axf_llama_generate_ex(m, prompt, n_prompt, n_gen, out_tokens, use_graph, 1);
}

int axf_llama_generate_ex(axf_llama* m, const int32_t* prompt, int n_prompt, int n_gen,
                          int32_t* out_tokens, int use_graph, int batched_prefill) {
    LL_LOADED(m);
    if (!prompt || n_prompt <= 0 || n_gen < 0 || (n_gen && !out_tokens))
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_generate: bad arguments");
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= m->hp.n_vocab)
            return fail(AXF_ERR_INVALID_ARG, "axf_llama_generate: prompt token out of range");
    // the reference emits a token only while n_past < n_ctx (:1613), n_past
    // starting at n_prompt: at most n_ctx - n_prompt tokens.  Asking for more
    // is an error here rather than a shorter result.
    if (n_prompt > m->hp.n_ctx || n_gen > m->hp.n_ctx - n_prompt)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_generate: context too long");
    hipStream_t st = m->ctx->stream;
    LL_HIP(launch_set_int(m->d_step, 0, st));
    LL_HIP(launch_set_int(m->d_pos, 0, st));
    if (use_graph) LL_TRY(ensure_graph(m, 0));
    if (batched_prefill && n_prompt > 1) {
        // llama_generate_cpu_impl (:1568-1576): one batch for the whole prompt;
        // the argmax of its last row is token 0, decoding continues at n_prompt
        LL_TRY(forward_batch(m, prompt, n_prompt, 0));
        LL_HIP(launch_argmax(m->d_token, m->arg_v, m->arg_i, m->logits, m->hp.n_vocab, nullptr,
                             nullptr, nullptr, st));
        LL_HIP(launch_set_int(m->d_pos, n_prompt, st));
    } else {
        // prefill token by token; the argmax of the last prompt step is token 0
        for (int t = 0; t < n_prompt; t++) {
            LL_HIP(launch_set_int(m->d_token, prompt[t], st));
            if (use_graph)
                LL_HIP(hipGraphLaunch(m->exec[0], st));
            else
                LL_HIP(enqueue_step(m, true, 0, 0, true));
        }
    }
    LL_HIP(launch_set_int(m->d_step, 0, st));
    if (n_gen > 0) LL_HIP(launch_push_token(m->d_tokens, m->d_step, m->d_token, st));
    for (int i = 1; i < n_gen; i++) {
        if (use_graph)
            LL_HIP(hipGraphLaunch(m->exec[0], st));
        else
            LL_HIP(enqueue_step(m, true, 0, 0, true));
    }
    if (n_gen > 0)
        LL_HIP(hipMemcpyAsync(out_tokens, m->d_tokens, (size_t)n_gen * 4, hipMemcpyDeviceToHost,
                              st));
    LL_HIP(hipStreamSynchronize(st));
    return AXF_OK;
}

int axf_llama_generate_sampled(axf_llama* m, const int32_t* prompt, int n_prompt,
                               int max_new_tokens, const axf_sampling* s, int32_t* out,
                               int* n_out, int use_graph) {
    LL_LOADED(m);
    if (!prompt || n_prompt <= 0 || max_new_tokens < 0 || !s || !n_out ||
        (max_new_tokens && !out))
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_generate_sampled: bad arguments");
    *n_out = 0;
    const auto& hp = m->hp;
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= hp.n_vocab)
            return fail(AXF_ERR_INVALID_ARG, "axf_llama_generate_sampled: prompt token out of range");
    if (n_prompt > hp.n_ctx)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_generate_sampled: prompt longer than the context");
    const int n_cand = sample_candidates(hp.n_vocab, sample_k(*s, hp.n_vocab));
    if (n_cand == 0)
        return fail(AXF_ERR_UNSUPPORTED,
                    "axf_llama_generate_sampled: top_k too large for the device sampler");
    // tokens are emitted while n_past < n_ctx (llama_model.cpp:1613); n_past
    // starts at n_prompt
    int n_gen = hp.n_ctx - n_prompt;
    if (n_gen > max_new_tokens) n_gen = max_new_tokens;
    if (n_gen <= 0) return AXF_OK;
    LL_TRY(sampler_alloc(m, n_cand));
    hipStream_t st = m->ctx->stream;
    std::vector<float> r((size_t)n_gen, 0.f);
    if (s->temperature > 0.f) sampling_uniforms(s->seed, r.data(), n_gen);
    LL_HIP(hipMemcpyAsync(m->d_r, r.data(), r.size() * 4, hipMemcpyHostToDevice, st));
    LL_HIP(hipMemcpyAsync(m->d_hist, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice, st));
    LL_HIP(launch_set_int(m->d_hist_n, n_prompt, st));
    LL_HIP(launch_set_int(m->d_step, 0, st));
    if (use_graph) LL_TRY(ensure_graph(m, 2, s));
    // prefill: one batch for a multi-token prompt (:1568-1576), else the
    // single-token forward (its greedy pick is overwritten below)
    if (n_prompt > 1)
        LL_TRY(forward_batch(m, prompt, n_prompt, 0));
    else
        LL_HIP(enqueue_step(m, false, prompt[0], 0, false));
    LL_HIP(launch_set_int(m->d_pos, n_prompt, st));
    // token 0: penalty over the prompt, sample with draw 0 (:1607-1609)
    LL_HIP(enqueue_pick(m, true, false, s));
    for (int i = 1; i < n_gen; i++) {
        if (use_graph)
            LL_HIP(hipGraphLaunch(m->exec[2], st));
        else
            LL_HIP(enqueue_step(m, true, 0, 0, true, s));
    }
    LL_HIP(hipMemcpyAsync(out, m->d_tokens, (size_t)n_gen * 4, hipMemcpyDeviceToHost, st));
    LL_HIP(hipStreamSynchronize(st));
    int n = n_gen;
    for (int i = 0; i < n_gen; i++)
        if (out[i] == s->eos_id) {  // stops before EOS; EOS is not emitted (:1612)
            n = i;
            break;
        }
    *n_out = n;
    return AXF_OK;
}

int axf_llama_bench_stage(axf_llama* m, int stage, int pos, int reps, float* ms) {
    LL_LOADED(m);
    if (!ms || stage < 1 || stage > 6 || pos < 0 || pos >= m->hp.n_ctx || reps <= 0)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_bench_stage: bad arguments");
    hipStream_t st = m->ctx->stream;
    LL_HIP(launch_set_int(m->d_pos, pos, st));
    LL_HIP(launch_set_int(m->d_token, 1, st));
    // one pass: the stage of every layer in turn (each layer's weights are
    // their own memory, so consecutive launches stream different bytes), or
    // n_layer head launches
    auto pass = [&]() -> hipError_t {
        for (int l = 0; l < m->hp.n_layer; l++) {
            const hipError_t e = stage == 6 ? head_pass(m, st)
                                            : enqueue_layer(m, l, m->d_pos, 0, stage, stage);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    };
    hipGraph_t g = nullptr;
    hipGraphExec_t ex = nullptr;
    if (!m->ctx->bench_eager) {
        LL_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        const hipError_t e = pass();
        const hipError_t e2 = hipStreamEndCapture(st, &g);
        if (e != hipSuccess || e2 != hipSuccess) {
            if (g) (void)hipGraphDestroy(g);
            return hip_fail(e != hipSuccess ? e : e2, "axf_llama_bench_stage");
        }
        const hipError_t e3 = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        if (e3 != hipSuccess) {
            (void)hipGraphDestroy(g);
            return hip_fail(e3, "axf_llama_bench_stage");
        }
    }
    auto run = [&]() -> hipError_t { return ex ? hipGraphLaunch(ex, st) : pass(); };
    hipError_t e = run();  // untimed
    if (e == hipSuccess) e = hipEventRecord(m->ctx->ev0, st);
    for (int r = 0; r < reps && e == hipSuccess; r++) e = run();
    if (e == hipSuccess) e = hipEventRecord(m->ctx->ev1, st);
    if (e == hipSuccess) e = hipEventSynchronize(m->ctx->ev1);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, m->ctx->ev0, m->ctx->ev1);
    if (ex) (void)hipGraphExecDestroy(ex);
    if (g) (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "axf_llama_bench_stage");
    return AXF_OK;
}

int axf_llama_bench_decode(axf_llama* m, int pos, int warmup, int steps, float* ms) {
    LL_LOADED(m);
    if (!ms || pos < 0 || pos >= m->hp.n_ctx || warmup < 0 || steps <= 0)
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_bench_decode: bad arguments");
    hipStream_t st = m->ctx->stream;
    const bool eager = m->ctx->bench_eager != 0;  // direct launches (profilers)
    if (!eager) LL_TRY(ensure_graph(m, 1));
    LL_HIP(launch_set_int(m->d_pos, pos, st));
    LL_HIP(launch_set_int(m->d_token, 1, st));
    auto step = [&]() -> hipError_t {
        return eager ? enqueue_step(m, true, 0, 0, false) : hipGraphLaunch(m->exec[1], st);
    };
    for (int i = 0; i < warmup; i++) LL_HIP(step());
    LL_HIP(hipEventRecord(m->ctx->ev0, st));
    for (int i = 0; i < steps; i++) LL_HIP(step());
    LL_HIP(hipEventRecord(m->ctx->ev1, st));
    LL_HIP(hipEventSynchronize(m->ctx->ev1));
    LL_HIP(hipEventElapsedTime(ms, m->ctx->ev0, m->ctx->ev1));
    return AXF_OK;
}

}  // extern "C"
