/*
 * axf_hip.h — C-ABI of the MI355X (gfx950) quantized decode path.
 *
 * Shared library: llm_core_amd/lib/libaxf_hip.so
 *
 * Conventions
 *   - Every entry point returns int: AXF_OK (0) or a negative AXF_ERR_* code;
 *     axf_hip_last_error() returns the message of the calling thread's last
 *     failure.  The C++ backend (llm_core_amd/csrc/host/hip_backend.cpp)
 *     turns non-zero codes into std::runtime_error, as the reference's CUDA
 *     backend does with check_cuda (src/backend/cuda/cuda_backend.cu:15-25).
 *   - One axf_ctx = one device + one in-order HIP stream.  Kernel entry points
 *     enqueue asynchronously on that stream; axf_hip_sync and the d2h copy
 *     block.  Pointer arguments named W, x, y, xq8, ... are device pointers
 *     owned by the caller (allocated with axf_hip_alloc or any HIP allocator).
 *   - Weights are GGUF super-blocks in their native layout: Q4_K 144 B and
 *     Q6_K 210 B per 256 weights (reference include/axonforge/dtype.hpp:136-155),
 *     rows contiguous, row r at W + r*row_bytes.
 *   - Q8_0 activations use the reference's block_q8_0: fp32 d followed by
 *     32 int8 (36 B per 32 values; src/backend/cpu_x86/kernels/q8_block.hpp:8-15).
 *   - y is overwritten (not accumulated) unless stated.
 *   - Alignment: W 16-byte aligned with row_bytes % 16 == 0 for Q4_K; W 4-byte
 *     aligned with row_bytes even for Q6_K; f32 vectors 16-byte aligned;
 *     Q8_0 buffers 4-byte aligned.  Violations return AXF_ERR_INVALID_ARG.
 */
#ifndef AXF_HIP_H
#define AXF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AXF_OK 0
#define AXF_ERR_INVALID_ARG (-1)
#define AXF_ERR_HIP (-2)
#define AXF_ERR_UNSUPPORTED (-3)
#define AXF_ERR_NO_DEVICE (-4)
#define AXF_ERR_STATE (-5)

/* GGML tensor type ids (reference dtype.hpp:107-124: 12 -> Q4_K_M, 14 -> Q6_K). */
#define AXF_TYPE_F32 0
#define AXF_TYPE_F16 1
#define AXF_TYPE_Q5_0 6
#define AXF_TYPE_Q8_0 8
#define AXF_TYPE_Q4_K 12
#define AXF_TYPE_Q6_K 14

typedef struct axf_ctx axf_ctx;

/* ---- errors / version ---------------------------------------------------- */
const char* axf_hip_last_error(void);
int axf_hip_version(int* major, int* minor, int* patch);

/* ---- lifecycle: replaces CudaBackend::initialize / finalize / device_id
 *      (src/backend/cuda/cuda_backend.cu:137-165) ------------------------------ */
int axf_hip_device_count(int* count);
int axf_hip_create(int device, axf_ctx** out);
int axf_hip_destroy(axf_ctx* ctx);
int axf_hip_device_name(axf_ctx* ctx, char* buf, int buflen);

/* ---- memory: replaces IBackend::allocate / transfer / synchronize
 *      (include/axonforge/backend.hpp:51-60; cuda_backend.cu:166-182) ---------- */
int axf_hip_alloc(axf_ctx* ctx, size_t bytes, void** dptr);
int axf_hip_free(axf_ctx* ctx, void* dptr);
int axf_hip_memcpy_h2d(axf_ctx* ctx, void* dst, const void* src, size_t bytes); /* blocking */
int axf_hip_memcpy_d2h(axf_ctx* ctx, void* dst, const void* src, size_t bytes); /* blocking */
int axf_hip_memcpy_d2d(axf_ctx* ctx, void* dst, const void* src, size_t bytes); /* async */
int axf_hip_sync(axf_ctx* ctx);

/* ---- quantized weight path ---------------------------------------------- */

/* Q4_K rows -> fp32, bit-exact with the Q4_K branch of emb_lookup
 * (src/models/llama_model.cpp:899-928).  y has 256*n_blocks floats. */
int axf_hip_dequant_q4k(axf_ctx* ctx, float* y, const void* W, int64_t n_blocks);

/* Q6_K rows -> fp32, bit-exact with q6k_row_to_f32 (llama_model.cpp:560-592). */
int axf_hip_dequant_q6k(axf_ctx* ctx, float* y, const void* W, int64_t n_blocks);

/* fp32 -> Q8_0, bit-exact with quantize_q8_avx2
 * (src/backend/cpu_x86/kernels/quant_q8_avx2.cpp:33-84).  n % 32 == 0. */
int axf_hip_quantize_q8_0(axf_ctx* ctx, void* xq8, const float* x, int n);

/* Q4_K x F32 GEMV over all rows: replaces gemv_q4k_avx2_range
 * (gemv_q4k_avx2.cpp:230-238) called over [0, rows).  cols % 256 == 0. */
int axf_hip_gemv_q4k_f32(axf_ctx* ctx, float* y, const void* W, const float* x, int rows,
                         int cols, size_t row_bytes);

/* Q6_K x F32 GEMV: replaces gemv_q6k_avx2_range (gemv_q6k_avx2.cpp:236-244). */
int axf_hip_gemv_q6k_f32(axf_ctx* ctx, float* y, const void* W, const float* x, int rows,
                         int cols, size_t row_bytes);

/* Q4_K x Q8_0 GEMV (the decode hot kernel): replaces gemv_q4k_r8_avxvnni_range /
 * gemv_q4k_r8_avx2_range (gemv_q4k_r8_avxvnni.cpp:177-183, gemv_q4k_r8_avx2.cpp:248-254)
 * and gemv_q4k_q8_{avx2,avxvnni}_range (gemv_q4k_q8_avx2.cpp:242-252), as dispatched
 * by gemv_wt_q8 (llama_model.cpp:767-831).  Takes the native layout (no r8 repack).
 * accumulate != 0 adds into y (fuses the residual add of llama_model.cpp:1277,1324). */
int axf_hip_gemv_q4k_q8(axf_ctx* ctx, float* y, const void* W, const void* xq8, int rows,
                        int cols, size_t row_bytes, int accumulate);

/* Q6_K x Q8_0 GEMV: replaces gemv_q6k_q8_avx2_range (gemv_q6k_q8_avx2.cpp:195-205). */
int axf_hip_gemv_q6k_q8(axf_ctx* ctx, float* y, const void* W, const void* xq8, int rows,
                        int cols, size_t row_bytes, int accumulate);

/* Batched Q4_K x Q8_0 (chunked prefill / multi-sequence decode):
 * Y[t*rows + o] = W[o,:] . XQ8[t,:] for t < T, token-major like
 * gemm_q4k_q8_avx2_range (gemv_q4k_q8_avx2.cpp:257-346); XQ8 row t starts at
 * block t*(cols/32). */
int axf_hip_gemm_q4k_q8(axf_ctx* ctx, float* Y, const void* W, const void* XQ8, int rows,
                        int T, int cols, size_t row_bytes);
/* Batched Q6_K x Q8_0: Y[t*rows + o] = W[o,:] . XQ8[t,:], token-major; replaces
 * the per-token gemv_q6k_q8_avx2_range loop of gemm_wt_q8 for Q6_K weights
 * (llama_model.cpp:860-873). */
int axf_hip_gemm_q6k_q8(axf_ctx* ctx, float* Y, const void* W, const void* XQ8, int rows,
                        int T, int cols, size_t row_bytes);
/* The same GEMMs with the kernel chosen explicitly (no reference counterpart;
 * for tests and measurement): path 0 automatic (1 below 8 tokens, 3 up to 64,
 * 2 above), 1 the dot4 kernel, 2 the matrix-core (int8 MFMA) kernel with an
 * LDS ring, 3 the int8 MFMA kernel with the weights loaded straight into
 * registers and split-K partial sums (Q4_K, T <= 64, 16-byte aligned W, XQ8
 * and row_bytes; otherwise as 2).  Results of the kernels differ only in float
 * summation order.  Q6_K takes the matrix cores
 * only where the last row's last block ends on a 16-byte boundary, under 2 GiB
 * from W (true of a 16-byte aligned W with row_bytes = cols / 256 * 210 and
 * rows * cols / 256 a multiple of 8); other Q6_K matrices take the dot4 kernel
 * on every path. */
int axf_hip_gemm_q4k_q8_path(axf_ctx* ctx, float* Y, const void* W, const void* XQ8, int rows,
                             int T, int cols, size_t row_bytes, int path);
int axf_hip_gemm_q6k_q8_path(axf_ctx* ctx, float* Y, const void* W, const void* XQ8, int rows,
                             int T, int cols, size_t row_bytes, int path);
/* As axf_hip_gemm_q4k_q8, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The matrix-core paths'
 * scratch (activation re-layout, or split-K partials) goes to a fixed 8 MiB
 * device array inside the library (one per GPU, held until the process ends)
 * instead of the context's hipMalloc'd scratch; this call allocates nothing.
 * Where path 0's kernel needs more than 8 MiB the LDS-ring kernel (path 2)
 * runs; token counts whose re-layout exceeds 8 MiB even there (T > 320 at
 * cols 11008, T > 896 at cols 4096) are AXF_ERR_INVALID_ARG.  Every call on one GPU shares the array: calls whose
 * kernels overlap on one GPU (other streams or contexts) race. */
int axf_hip_gemm_q4k_q8_noalloc(axf_ctx* ctx, float* Y, const void* W, const void* XQ8,
                                int rows, int T, int cols, size_t row_bytes);

/* Other GGUF weight types of the decode path (LM heads of Qwen / DeepSeek files,
 * F16 models).  cols is a multiple of 32 for the block types, rows of
 * cols/32 blocks (34 B Q8_0: fp16 d + 32 int8; 22 B Q5_0: fp16 d, u32 high
 * bits, 16 B nibbles), 2-byte aligned.
 * Q8_0 x Q8_0: replaces gemv_q8_0_weight_q8 / q8_0_weight_dot_q8_row
 * (llama_model.cpp:171-228), the q8_fast branch of gemv_wt_q8 (:825-828). */
int axf_hip_gemv_q8_0w_q8(axf_ctx* ctx, float* y, const void* W, const void* xq8, int rows,
                          int cols, size_t row_bytes, int accumulate);
/* Q8_0 x fp32: q8_0_weight_dot_row (:154-169) in gemv_wt (:701-712); x 16-byte aligned. */
int axf_hip_gemv_q8_0w_f32(axf_ctx* ctx, float* y, const void* W, const float* x, int rows,
                           int cols, size_t row_bytes);
/* Q5_0 x fp32: q5_0_dot_row (:245-267) in gemv_wt (:713-724). */
int axf_hip_gemv_q5_0_f32(axf_ctx* ctx, float* y, const void* W, const float* x, int rows,
                          int cols, size_t row_bytes);
/* F16 x fp32 (+ bias b, may be NULL): gemv_f16_avx2_range (gemv_f16_avx2.cpp:138-153);
 * W rows of cols halfs, W and x 16-byte aligned, cols % 8 == 0. */
int axf_hip_gemv_f16_f32(axf_ctx* ctx, float* y, const void* W, const float* x, const float* b,
                         int rows, int cols);
/* T-token product with fp32 token rows for Q8_0 / Q5_0 / F16 weights (qtype
 * AXF_TYPE_Q8_0, AXF_TYPE_Q5_0 or AXF_TYPE_F16): Y[t*rows + o] (+= when
 * accumulate) sum_k W[o][k] X[t*cols + k].  Replaces gemm_wt_q8's fallback in
 * the batched prefill (llama_model.cpp:876-879), which runs gemv_wt (:670-731)
 * on each token's fp32 row; each weight block is dequantised once per 16 or 32
 * tokens here.  cols % 32 == 0; X and Y 4-byte aligned; F16: W 16-byte aligned
 * and row_bytes a multiple of 16 (2*cols for packed rows). */
int axf_hip_gemm_misc_f32(axf_ctx* ctx, int qtype, float* Y, const void* W, const float* X,
                          int rows, int T, int cols, size_t row_bytes, int accumulate);

/* Greedy pick: *idx_dev = first index of the maximum of x[0..n), the
 * std::max_element of sample() (llama_model.cpp:1470-1471).  idx_dev is a
 * device int. */
int axf_hip_argmax_f32(axf_ctx* ctx, int* idx_dev, const float* x, int n);

/* Sampling parameters of LlamaConfig (include/axonforge/models/llama.hpp:18-33). */
typedef struct {
    float temperature;      /* <= 0: greedy (std::max_element) */
    int top_k;              /* <= 0 or >= n_vocab: the whole vocabulary */
    float top_p;            /* 1: no nucleus cut */
    float rep_penalty;      /* 1: no repetition penalty */
    int rep_penalty_last_n; /* window of the penalty */
    uint32_t seed;          /* std::mt19937 seed; the reference uses 42 */
    int32_t eos_id;         /* generation stops before this token; -1: none */
} axf_sampling;

/* One token choice: the reference's apply_rep_penalty over the last
 * rep_penalty_last_n of hist[0..n_hist) (llama_model.cpp:1595-1605; applied to
 * logits_dev in place, as the reference does to state.logits), then sample()
 * (:1466-1498) with the uniform draw r.  *token (host) receives the id.  Any
 * top_k: up to 16384 candidates (ceil(n_vocab / 4096) * min(k, 4096)) are
 * sorted in LDS, more (e.g. top_k above 431 at n_vocab 151936, or the whole
 * vocabulary) in place in device memory by one workgroup, a few ms per call.
 * Among exactly equal scores the lower index ranks first. */
int axf_hip_sample(axf_ctx* ctx, float* logits_dev, int n_vocab, const axf_sampling* s,
                   const int32_t* hist, int n_hist, float r, int32_t* token);
/* The reference's random stream: the first n outputs of std::mt19937(seed), and
 * the first n std::uniform_real_distribution<float>(0, 1) draws from it as
 * libstdc++ computes them (one 32-bit output each). */
int axf_mt19937(uint32_t seed, uint32_t* out, int n);
int axf_sampling_uniforms(uint32_t seed, float* out, int n);

/* ---- decode-step operations (llama_forward_token, llama_model.cpp:1207-1333) */

/* y = w*(x*s), s = 1/sqrt(mean(x^2)+eps): rms_norm_out (llama_model.cpp:396-419).
 * y and/or yq8 (Q8_0 of the result) may be NULL.  n % 32 == 0. */
int axf_hip_rmsnorm(axf_ctx* ctx, float* y, void* yq8, const float* x, const float* w, int n,
                    float eps);

/* Host: RopeCache::build (llama_model.cpp:1031-1043), tables [max_pos][head_dim/2]. */
int axf_rope_table(float* cos_t, float* sin_t, int head_dim, float theta, int max_pos);

/* Rotate-half RoPE with a device cos/sin table: apply_rope / rope_and_store_k
 * (llama_model.cpp:1046-1080).  dst may equal src. */
int axf_hip_rope(axf_ctx* ctx, float* dst, const float* src, int pos, int n_heads,
                 int head_dim, const float* cos_t, const float* sin_t);

/* Single-token GQA attention over an fp32 KV cache whose rows are
 * n_kv_heads*head_dim floats (llama_model.cpp:1255-1272); seq = positions
 * 0..seq-1 used.  outq8 (Q8_0 of out) may be NULL.  head_dim in {64,128,256}. */
int axf_hip_attn_decode(axf_ctx* ctx, float* out, void* outq8, const float* q,
                        const float* kcache, const float* vcache, int seq, int n_heads,
                        int n_kv_heads, int head_dim);
/* Causal attention of T query rows at positions pos0 .. pos0+T-1, the
 * multi-token attention of llama_forward_batch (llama_model.cpp:1410-1426):
 * row t (at q + t*q_ld, n_heads*head_dim raw projections) gets the bias bq
 * (may be NULL) and RoPE from the tables (cos_t/sin_t [n_pos][head_dim/2]),
 * then attends to cache rows 0 .. pos0+t (K rows already RoPE'd).  out row t
 * at out + t*n_heads*head_dim; outq8 (may be NULL) holds its Q8_0 blocks.
 * path 0: the matrix-core kernel (what the decoder's prefill uses); 1: the
 * decode split/combine kernels over a token grid (no reference counterpart;
 * for comparison). */
int axf_hip_attn_prefill(axf_ctx* ctx, float* out, void* outq8, const float* q, int q_ld,
                         const float* bq, const float* kcache, const float* vcache, int pos0,
                         int T, int n_heads, int n_kv_heads, int head_dim, const float* cos_t,
                         const float* sin_t, int path);

/* out = silu(gate)*up as swiglu_avx2 (llama_model.cpp:348-368); out may equal
 * gate; outq8 may be NULL.  n % 32 == 0. */
int axf_hip_swiglu(axf_ctx* ctx, float* out, void* outq8, const float* gate, const float* up,
                   int n);

/* y = a + b (residual add, llama_model.cpp:1277). */
int axf_hip_add(axf_ctx* ctx, float* y, const float* a, const float* b, int n);

/* out = dequantised row `token` (0 <= token < rows) of a Q4_K/Q6_K matrix
 * (emb_lookup, llama_model.cpp:882-934). */
int axf_hip_embed(axf_ctx* ctx, float* out, int qtype, const void* W, int token, int rows,
                  int cols);

/* ---- timing (stream-ordered HIP events on the context stream) ----------- */
int axf_hip_timer_start(axf_ctx* ctx);
int axf_hip_timer_stop(axf_ctx* ctx, float* ms); /* waits for the stop event */

/* Benchmark helper (no reference counterpart): captures one HIP graph of n_w
 * GEMV launches, launch i reading weight copy W_list[i] (so consecutive
 * launches stream different memory), replays it once untimed and then `reps`
 * times between two events; *ms = elapsed milliseconds for reps*n_w launches.
 * kind: 0 Q4_K x Q8_0, 1 Q6_K x Q8_0, 2 Q4_K x F32, 3 Q6_K x F32. */
int axf_hip_bench_gemv(axf_ctx* ctx, int kind, float* y, const void* const* W_list, int n_w,
                       const void* x, int rows, int cols, size_t row_bytes, int reps, float* ms);

/* Benchmark helper (no reference counterpart): a plain streaming read of
 * `bytes` (a multiple of 16) from each of the n device buffers in turn,
 * reps times over the list, as axf_hip_bench_gemv times its GEMVs; unroll
 * (1, 2, 4, 8) 16-byte loads in flight per thread, wgs workgroups of 256
 * threads.  *ms = elapsed milliseconds of the timed passes.  It measures what
 * one launch of a given size can read, the ceiling the GEMVs are compared to. */
int axf_hip_bench_read(axf_ctx* ctx, const void* const* bufs, int n, size_t bytes, int unroll,
                       int wgs, int reps, float* ms);
/* Benchmark helpers (no reference counterpart): eager != 0 makes
 * axf_hip_bench_gemv, axf_hip_bench_gemm and axf_llama_bench_decode on this
 * context launch every kernel directly instead of capturing and replaying a
 * HIP graph (for runs under a profiler; the timings then include the host's
 * launch gaps). */
int axf_hip_bench_set_eager(axf_ctx* ctx, int eager);
/* Benchmark helper (no reference counterpart): as axf_hip_bench_gemv for the
 * T-token GEMM of axf_hip_gemm_q4k_q8 / axf_hip_gemm_q6k_q8 (qtype AXF_TYPE_Q4_K or
 * AXF_TYPE_Q6_K weights, Q8_0 activations); path as for axf_hip_gemm_q4k_q8_path. */
int axf_hip_bench_gemm(axf_ctx* ctx, int qtype, float* Y, const void* const* W_list, int n_w,
                       const void* XQ8, int rows, int T, int cols, size_t row_bytes, int path,
                       int reps, float* ms);

/* ---- synthetic GGUF weights (host code, deterministic) ------------------ */
/* dst[i] ~ N(mean, std) from a counter-based generator (splitmix64 + Box-Muller);
 * element i depends only on (seed, i). */
int axf_synth_normal(float* dst, int64_t n, uint64_t seed, float mean, float stddev);
/* fp32 -> GGUF blocks (qtype AXF_TYPE_Q4_K or AXF_TYPE_Q6_K), n % 256 == 0. */
int axf_synth_quantize(int qtype, uint8_t* dst, const float* src, int64_t n);
/* rows x cols matrix drawn N(0, std) and quantized, written row-major in GGUF
 * layout; multi-threaded, result independent of the thread count. */
int axf_synth_weight(int qtype, uint8_t* dst, int64_t rows, int64_t cols, uint64_t seed,
                     float stddev);
size_t axf_row_bytes(int qtype, int64_t cols);

/* ---- GGUF v2/v3 files (GgufReader, src/loader/gguf_reader.hpp and
 *      gguf_loader.cpp:49-335; host code, no GPU needed) --------------------- */
typedef struct axf_gguf axf_gguf;

/* Replaces GgufReader::open + parse (gguf_loader.cpp:49-163): mmap the file and
 * parse header, KV pairs and tensor infos.  Format errors return
 * AXF_ERR_INVALID_ARG with the reference's runtime_error message ("GgufReader:
 * invalid magic (not a GGUF file)", "... unsupported GGUF version N (supported:
 * 2, 3)", "... unexpected end of file (truncated)", ...). */
int axf_gguf_open(const char* path, axf_gguf** out);
int axf_gguf_close(axf_gguf* g);
uint32_t axf_gguf_version(const axf_gguf* g);      /* GgufReader::version */
uint64_t axf_gguf_alignment(const axf_gguf* g);    /* general.alignment (u32) or 32 */
uint64_t axf_gguf_data_offset(const axf_gguf* g);  /* tensor_data_offset */
uint64_t axf_gguf_file_size(const axf_gguf* g);
int64_t axf_gguf_n_kv(const axf_gguf* g);
int64_t axf_gguf_n_tensors(const axf_gguf* g);
/* KV access with the reference's typed accessors and coercions
 * (gguf_loader.cpp:222-296): a missing key, or a stored type that the
 * accessor does not convert, returns def.  axf_gguf_kv_type gives the value
 * type tag (0 u8 .. 12 f64, 8 string, 9 array) or -1. */
int axf_gguf_kv_type(const axf_gguf* g, const char* key);
uint64_t axf_gguf_get_u64(const axf_gguf* g, const char* key, uint64_t def);
uint32_t axf_gguf_get_u32(const axf_gguf* g, const char* key, uint32_t def);
int32_t axf_gguf_get_i32(const axf_gguf* g, const char* key, int32_t def);
float axf_gguf_get_f32(const axf_gguf* g, const char* key, float def);
int axf_gguf_get_bool(const axf_gguf* g, const char* key, int def);
/* string value; *s stays valid until axf_gguf_close */
int axf_gguf_get_str(const axf_gguf* g, const char* key, const char** s, size_t* len);
uint64_t axf_gguf_get_array_count(const axf_gguf* g, const char* key);
int axf_gguf_get_array_type(const axf_gguf* g, const char* key); /* element tag or -1 */
int axf_gguf_get_array_str(const axf_gguf* g, const char* key, uint64_t i, const char** s,
                           size_t* len);
int axf_gguf_get_array_data(const axf_gguf* g, const char* key, const void** data,
                            size_t* bytes);

typedef struct {
    const char* name;   /* valid until axf_gguf_close */
    int n_dims;
    int64_t shape[4];   /* GGML order: shape[0] is the innermost (columns) */
    int ggml_type;      /* 0 F32, 12 Q4_K, 14 Q6_K, ... (the AXF_TYPE_* values) */
    uint64_t offset;    /* within the data blob */
    uint64_t nbytes;    /* gguf_tensor_nbytes; 0 for types the reference does not size */
    const void* data;   /* into the mapping; NULL when the range leaves the file */
} axf_gguf_tensor;
/* GgufReader::tensor_info / weight_tensor (zero-copy view). */
int axf_gguf_tensor_info(const axf_gguf* g, int64_t i, axf_gguf_tensor* out);
int64_t axf_gguf_find_tensor(const axf_gguf* g, const char* name); /* index or -1 */
/* gguf_tensor_nbytes over ggml_type_to_dtype (include/axonforge/dtype.hpp:107-155)
 * and gguf_type_pod_size (:87-104). */
size_t axf_gguf_type_nbytes(int ggml_type, int64_t numel);
size_t axf_gguf_pod_size(int type_tag);

/* ModelConfig of Engine::from_gguf (src/engine.cpp:79-118): <arch>.block_count,
 * .embedding_length, .feed_forward_length, .attention.head_count(_kv),
 * .context_length (default 4096), .attention.layer_norm_rms_epsilon (1e-5),
 * .rope.freq_base (10000), .rope.scaling.alpha (hunyuan-dense theta scaling),
 * vocabulary = length of tokenizer.ggml.tokens, BOS/EOS ids (defaults 1 / 2). */
typedef struct {
    char arch[64];
    int n_layer, n_embd, ffn_dim, n_heads, n_kv_heads, head_dim, max_seq_len, n_vocab;
    float rms_eps, rope_theta, rope_scaling_alpha;
    int weight_type; /* GGML type of the file's first tensor, -1 if none */
    int32_t bos_id, eos_id;
} axf_gguf_model_config;
int axf_gguf_read_model_config(const axf_gguf* g, axf_gguf_model_config* out);

/* ---- LLaMA-family decoder on the device (llama_generate's `-b hip` hook,
 *      the model-level branch of llama_model.cpp:1633-1642) ----------------- */
typedef struct axf_llama axf_llama;

typedef struct {
    int n_layer, n_embd, n_heads, n_kv_heads, ffn_dim, n_vocab, n_ctx;
    float rms_eps, rope_theta;
    /* QkNormOrder (llama_model.cpp:955-959, chosen from the architecture at
     * :1520-1522): 0 none, 1 per-head q/k RMSNorm before RoPE (qwen3), 2 after
     * RoPE (hunyuan-dense); the weights are blk.N.attn_{q,k}_norm.weight
     * (head_dim floats, optional as in the reference) */
    int qk_norm_order;
} axf_llama_hparams;

/* n_embd and ffn_dim multiples of 32 (n_embd <= 8192, ffn_dim <= 32768),
 * head_dim = n_embd / n_heads of 64, 128 or 256, at most 8 query heads per
 * KV head, n_ctx <= 32768; otherwise AXF_ERR_UNSUPPORTED (or
 * AXF_ERR_INVALID_ARG for inconsistent values). */
int axf_llama_create(axf_ctx* ctx, const axf_llama_hparams* hp, axf_llama** out);
int axf_llama_destroy(axf_llama* m);
/* Register a host tensor by its GGUF name (token_embd.weight, output_norm.weight,
 * output.weight, blk.N.{attn_norm,ffn_norm,attn_q,attn_k,attn_v,attn_output,
 * ffn_gate,ffn_up,ffn_down}.weight, optional blk.N.attn_{q,k,v}.bias and, with
 * qk_norm_order != 0, blk.N.attn_{q,k}_norm.weight).  The host
 * buffer must stay valid until axf_llama_load returns. */
int axf_llama_set_tensor(axf_llama* m, const char* name, int qtype, const void* host,
                         size_t bytes);
/* Upload all registered tensors once and allocate the KV cache and buffers.
 * Every matrix may be Q4_K or Q6_K (rows of whole 256-weight super-blocks),
 * Q8_0 or Q5_0 (rows of whole 32-blocks) or F16 (rows a multiple of 8), in
 * any mix: the decode step multiplies Q4_K / Q6_K / Q8_0 matrices with the
 * Q8_0 activation and Q5_0 / F16 ones with the fp32 activation (gemv_wt_q8,
 * llama_model.cpp:767-831); the batched prefill gives Q8_0 / Q5_0 / F16 the
 * fp32 rows (gemm_wt_q8, :837-879).  Another type: AXF_ERR_UNSUPPORTED. */
int axf_llama_load(axf_llama* m);
/* Register every model tensor of an open GGUF file (the names build_weights
 * reads, llama_model.cpp:975-1006) straight from the mapping and load.  F32
 * vectors; F16, Q8_0, Q5_0, Q4_K and Q6_K matrices (as axf_llama_load). */
int axf_llama_load_gguf(axf_llama* m, const axf_gguf* g);
/* Engine::from_gguf + the model construction of llama_generate_cpu_impl
 * (llama_model.cpp:1508-1522): hyperparameters from the file's metadata with
 * the reference's defaults, the q/k norm order from the architecture, context = min(context_length, max_context_len)
 * (max_context_len <= 0: 4096, LlamaConfig's default), weights uploaded from
 * the mapping.  The file is closed before returning. */
int axf_llama_from_gguf(axf_ctx* ctx, const char* path, int max_context_len, axf_llama** out);
size_t axf_llama_device_bytes(axf_llama* m);
/* The hyperparameters the model was created with (no reference counterpart;
 * for callers of axf_llama_from_gguf). */
int axf_llama_get_hparams(const axf_llama* m, axf_llama_hparams* hp);
/* Residual stream / KV access (host buffers). */
int axf_llama_set_x(axf_llama* m, const float* x);
int axf_llama_get_x(axf_llama* m, float* x);
int axf_llama_set_kv(axf_llama* m, int layer, const float* k, const float* v, int n_pos);
int axf_llama_fill_kv_random(axf_llama* m, int n_pos, uint64_t seed);
int axf_llama_get_logits(axf_llama* m, float* logits);
/* One decoder layer at `pos` on the residual stream (eager). */
int axf_llama_forward_layer(axf_llama* m, int layer, int pos);
/* Stages first..last (1 <= first <= last <= 5) of one decoder layer at `pos`,
 * eager, with the kernels the decode step runs: 1 the q|k|v projections of
 * RMSNorm(x) * attn_norm (before bias), 2 attention (bias and RoPE of q and k,
 * K/V row `pos` stored, output and its Q8_0), 3 o projection and x +=, 4
 * gate|up of RMSNorm(x) * ffn_norm and SwiGLU, 5 down projection of Q8_0(h)
 * and x +=.  The stages of llama_forward_token's layer body
 * (llama_model.cpp:1222-1325); no reference counterpart as an entry point:
 * it exists so parity tests can check each fused kernel on its own. */
int axf_llama_forward_layer_stages(axf_llama* m, int layer, int pos, int first, int last);
/* Read back a decoder buffer (the device counterparts of LlamaState's s.x,
 * s.q|s.k|s.v, s.attn_out, xq8 and s.gate, llama_model.cpp:1096-1166).
 * `bytes` must equal the buffer's size:
 *   X        n_embd floats (residual stream)
 *   QKV      (n_heads + 2 n_kv_heads) * head_dim floats: q|k|v projections
 *            before bias and RoPE, as written by stage 1
 *   ATTN     n_heads * head_dim floats: attention output (stage 2)
 *   ATTN_Q8  its Q8_0 blocks, n_heads * head_dim / 32 * 36 bytes
 *   H        ffn_dim floats: SwiGLU output (stage 4)
 *   LOGITS   n_vocab floats */
enum {
    AXF_LLAMA_BUF_X = 0,
    AXF_LLAMA_BUF_QKV = 1,
    AXF_LLAMA_BUF_ATTN = 2,
    AXF_LLAMA_BUF_ATTN_Q8 = 3,
    AXF_LLAMA_BUF_H = 4,
    AXF_LLAMA_BUF_LOGITS = 5
};
int axf_llama_get_buffer(axf_llama* m, int which, void* out, size_t bytes);
/* KV cache rows pos0..pos0+n_pos-1 of a layer (K after RoPE, as stored). */
int axf_llama_get_kv(axf_llama* m, int layer, float* k, float* v, int pos0, int n_pos);
/* Full single-token forward (embedding .. logits), eager. */
int axf_llama_forward_token(axf_llama* m, int token, int pos);
/* Batched prefill: replaces llama_forward_batch (llama_model.cpp:1339-1462).
 * Runs tokens[0..T) at positions pos_start..pos_start+T-1 (K/V rows written),
 * the projections as T-token GEMMs (matrix cores from 8 tokens up), causal
 * attention per row; leaves the last row's logits (get_logits) and,
 * as the reference leaves s.x, that row after the final RMSNorm (get_x).
 * Long prompts run in chunks of up to 512 tokens. */
int axf_llama_forward_batch(axf_llama* m, const int32_t* tokens, int T, int pos_start);
/* Greedy generation (greedy loop of llama_generate_cpu_impl,
 * llama_model.cpp:1568-1624, without EOS): the prompt is prefilled as one batch
 * when n_prompt > 1 (as the reference does), then n_gen tokens are decoded.
 * use_graph != 0 replays one captured HIP graph per decode step.  The
 * reference stops at n_past >= n_ctx, i.e. after n_ctx - n_prompt tokens;
 * n_gen above that is AXF_ERR_INVALID_ARG. */
int axf_llama_generate(axf_llama* m, const int32_t* prompt, int n_prompt, int n_gen,
                       int32_t* out_tokens, int use_graph);
/* As axf_llama_generate; batched_prefill == 0 prefills token by token (the
 * llama_forward_token path) instead. */
int axf_llama_generate_ex(axf_llama* m, const int32_t* prompt, int n_prompt, int n_gen,
                          int32_t* out_tokens, int use_graph, int batched_prefill);
/* The generation loop of llama_generate_cpu_impl (llama_model.cpp:1590-1624)
 * with sampling on the device: the prompt (BOS already in place: the caller
 * prepends it as :1563-1566 does) is prefilled (one batch when n_prompt > 1),
 * then each step applies the repetition penalty over the prompt and the tokens
 * so far, samples (temperature / top-k / top-p, the uniform draws of
 * std::mt19937(s->seed) precomputed on the host) and decodes the token, one
 * captured HIP graph per step when use_graph != 0.  Stops before s->eos_id
 * (not emitted) and when the context is full; *n_out = tokens written to out
 * (at most max_new_tokens). */
int axf_llama_generate_sampled(axf_llama* m, const int32_t* prompt, int n_prompt,
                               int max_new_tokens, const axf_sampling* s, int32_t* out,
                               int* n_out, int use_graph);
/* Benchmark helper (no reference counterpart): mean milliseconds of `reps`
 * axf_llama_forward_batch calls on T synthetic tokens at positions 0..T-1,
 * after one untimed call (HIP events on the context stream). */
int axf_llama_bench_prefill(axf_llama* m, int T, int reps, float* ms);
/* Benchmark helper (no reference counterpart): one stage of the decode step
 * (1 q|k|v GEMV with the RMSNorm prologue, 2 attention split + combine, 3 o
 * GEMV with x +=, 4 gate|up GEMV with SwiGLU, 5 down GEMV with x +=, 6 the head
 * with the greedy pick) enqueued for layers 0..n_layer-1 in turn (stage 6:
 * n_layer times) at position `pos`, captured as one graph, replayed once
 * untimed and `reps` times between HIP events (direct launches under
 * axf_hip_bench_set_eager).  *ms = elapsed milliseconds of the reps passes.
 * The buffers the stages read hold whatever the last step left. */
int axf_llama_bench_stage(axf_llama* m, int stage, int pos, int reps, float* ms);
/* Time `steps` graph-replayed decode steps, each at position `pos` (the
 * attention reads KV rows 0..pos; rows below pos must already be filled, row
 * pos is rewritten by every step), after `warmup` untimed steps; each step
 * feeds the previous step's argmax.  *ms = elapsed milliseconds of the timed
 * steps (HIP events on the context stream). */
int axf_llama_bench_decode(axf_llama* m, int pos, int warmup, int steps, float* ms);

#ifdef __cplusplus
}
#endif
#endif
