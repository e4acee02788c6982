// gemv_misc.hip — GEMVs and embedding rows for the other GGUF weight types the
// reference's decode path handles (LM heads of Qwen / DeepSeek files and F16
// models), for gfx950:
//   * Q8_0 weights (34-byte blocks: fp16 d, 32 int8) x Q8_0 activations —
//     q8_0_weight_dot_q8_row (src/models/llama_model.cpp:171-211): per block
//     (d_w * d_x) * isum, isum the exact int32 dot (v_dot4_i32_i8);
//   * Q8_0 weights x fp32 activations — q8_0_weight_dot_row (:154-169);
//   * Q5_0 weights (22-byte blocks: fp16 d, u32 high bits, 16 B nibbles) x fp32
//     activations — q5_0_dot_row (:241-267): w = d * (q5 - 16);
//   * F16 weights x fp32 activations (+ optional bias) — gemv_f16_avx2_range
//     (src/backend/cpu_x86/kernels/gemv_f16_avx2.cpp:138-153);
//   * embedding rows of the three types — emb_lookup (:882-898), exact.
// These are HBM-bound streams.  LPR lanes share a row and stride over its
// 32-element blocks (F16: 8-element groups); the lane partials are reduced with
// shuffles, so the fp32 sums differ from the reference's sequential order
// only by reassociation.  gridDim.y tokens (the batched prefill): token t reads
// activation row t (cols floats, or cols/32 Q8_0 blocks) and writes y row t
// (rows floats); accumulate != 0 adds to y (the residual projections).  The 34- and 22-byte blocks are 2-byte aligned and
// read as 16-bit words; F16 rows are read 16 bytes at a time (the entry points
// require 16-byte aligned rows).
#include "common.hpp"

namespace axf {

namespace {

constexpr int kMiscThreads = 256;

__device__ __forceinline__ uint32_t ld2(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}

// 2-byte-aligned 32-bit word
__device__ __forceinline__ uint32_t ld2x2(const uint8_t* p) { return ld2(p) | (ld2(p + 2) << 16); }

template <int LPR>
__device__ __forceinline__ float lanes_sum(float v) {
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// One row per LPR lanes; blockIdx.x * (256 / LPR) + threadIdx.x / LPR is the row.
template <int LPR>
__device__ __forceinline__ long misc_row() {
    return (long)blockIdx.x * (kMiscThreads / LPR) + threadIdx.x / LPR;
}

// Row dots, shared by the token-grid GEMVs below and the fused decode stage
// kernel (activation in global memory or in LDS).  Lane rl of the row's LPR
// lanes takes blocks rl, rl + LPR, ...; the activation's 32-float (or 36-byte
// Q8_0) block b starts at float XS * b (XS = 32 in global memory, 36 in LDS,
// where the padding spreads the lanes' blocks over the banks).
template <int LPR>
__device__ __forceinline__ float dot_q8w_q8(const uint8_t* __restrict__ wr,
                                            const uint8_t* __restrict__ xq8, int nb, int rl) {
    float acc = 0.f;
    for (int b = rl; b < nb; b += LPR) {
        const uint8_t* wb = wr + (long)b * 34;
        const uint8_t* xb = xq8 + (long)b * Q8_0_BYTES;
        // the 34-byte block is 2-byte aligned: d as a 16-bit word, the 32 codes
        // from 8 aligned dwords starting at wb (sh = 0: d and codes 0..29) or
        // wb + 2 (sh = 2: codes 0..31) and the 16-bit word at wb + 32 (codes
        // 30, 31), joined by v_alignbyte; every byte read lies in the block
        const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(wb) & 3u);
        const uint8_t* wa = wb + sh;
        uint32_t w[9];
#pragma unroll
        for (int k = 0; k < 8; k++) w[k] = ld4(wa + 4 * k);
        w[8] = ld2(wb + 32);
        const float scale = h2f(ld2(wb)) * __uint_as_float(ld4(xb));
        int isum = 0;
#pragma unroll
        for (int k = 0; k < 8; k++)
            isum = dot4((int)alignbyte(w[k + 1], w[k], 2u - sh), (int)ld4(xb + 4 + 4 * k), isum);
        acc = fmaf(scale, (float)isum, acc);
    }
    return acc;
}

// bit j of the low 4 bits of s into bit 0 of byte j (the four products
// s << 0, 7, 14, 21 do not overlap, so the multiply has no carries)
__device__ __forceinline__ uint32_t spread4(uint32_t s) {
    return __umul24(s, 0x00204081u) & 0x01010101u;
}

// Q5_0: w = d * (q5 - 16), q5 = nibble | (bit of qh) << 4.  Per block the
// 32 products q5 * x are summed first and the block adds d * (sum - 16 * sx),
// sx = the block's sum of x (SX: precomputed at float XS * b + 32; else summed
// here): 4 q5 values are built per integer operation sequence as bytes and
// converted with v_cvt_f32_ubyte*, and x is read as float4.
template <int LPR, int XS, bool SX>
__device__ __forceinline__ float dot_q5_0_f32(const uint8_t* __restrict__ wr,
                                              const float* __restrict__ x, int nb, int rl) {
    float acc = 0.f;
    for (int b = rl; b < nb; b += LPR) {
        const uint8_t* wb = wr + (long)b * 22;
        const float d = h2f(ld2(wb));
        const uint32_t qh = ld2x2(wb + 2);
        const float* xb = x + XS * b;
        float s = 0.f, sx = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t qs = ld2x2(wb + 6 + 4 * k);  // bytes 4k..4k+3 of the 16
            // elements 4k..4k+3 (low nibbles) and 4k+16..4k+19 (high nibbles)
            const uint32_t lo = (qs & 0x0f0f0f0fu) | (spread4((qh >> (4 * k)) & 0xfu) << 4);
            const uint32_t hi = ((qs >> 4) & 0x0f0f0f0fu) | (spread4((qh >> (16 + 4 * k)) & 0xfu) << 4);
            const float4 xl = *reinterpret_cast<const float4*>(xb + 4 * k);
            const float4 xh = *reinterpret_cast<const float4*>(xb + 16 + 4 * k);
            s = fmaf((float)(lo & 0xffu), xl.x, s);
            s = fmaf((float)((lo >> 8) & 0xffu), xl.y, s);
            s = fmaf((float)((lo >> 16) & 0xffu), xl.z, s);
            s = fmaf((float)(lo >> 24), xl.w, s);
            s = fmaf((float)(hi & 0xffu), xh.x, s);
            s = fmaf((float)((hi >> 8) & 0xffu), xh.y, s);
            s = fmaf((float)((hi >> 16) & 0xffu), xh.z, s);
            s = fmaf((float)(hi >> 24), xh.w, s);
            if constexpr (!SX) sx += ((xl.x + xl.y) + (xl.z + xl.w)) + ((xh.x + xh.y) + (xh.z + xh.w));
        }
        if constexpr (SX) sx = xb[32];
        acc = fmaf(d, fmaf(-16.f, sx, s), acc);
    }
    return acc;
}

template <int LPR, int XS>
__device__ __forceinline__ float dot_f16_f32(const uint16_t* __restrict__ W,
                                             const float* __restrict__ x, int cols, int rl) {
    float acc = 0.f;
    const uint4* wr = reinterpret_cast<const uint4*>(W);
    const int ng = cols / 8;
    for (int g = rl; g < ng; g += LPR) {
        const uint4 w = wr[g];
        const float* xg = x + XS * (g >> 2) + 8 * (g & 3);
        const float4 x0 = reinterpret_cast<const float4*>(xg)[0];
        const float4 x1 = reinterpret_cast<const float4*>(xg)[1];
        acc = fmaf(h2f(w.x & 0xffffu), x0.x, acc);
        acc = fmaf(h2f(w.x >> 16), x0.y, acc);
        acc = fmaf(h2f(w.y & 0xffffu), x0.z, acc);
        acc = fmaf(h2f(w.y >> 16), x0.w, acc);
        acc = fmaf(h2f(w.z & 0xffffu), x1.x, acc);
        acc = fmaf(h2f(w.z >> 16), x1.y, acc);
        acc = fmaf(h2f(w.w & 0xffffu), x1.z, acc);
        acc = fmaf(h2f(w.w >> 16), x1.w, acc);
    }
    return acc;
}

template <int LPR>
__global__ __launch_bounds__(kMiscThreads) void k_gemv_q8w_q8(float* __restrict__ y,
                                                              const uint8_t* __restrict__ W,
                                                              const uint8_t* __restrict__ xq8,
                                                              int rows, int nb, long row_bytes,
                                                              int accumulate) {
    y += (size_t)blockIdx.y * rows;
    xq8 += (size_t)blockIdx.y * nb * Q8_0_BYTES;
    const long row = misc_row<LPR>();
    const int rl = threadIdx.x % LPR;
    float acc = 0.f;
    if (row < rows) acc = dot_q8w_q8<LPR>(W + row * row_bytes, xq8, nb, rl);
    acc = lanes_sum<LPR>(acc);
    if (row < rows && rl == 0) y[row] = accumulate ? y[row] + acc : acc;
}

template <int LPR>
__global__ __launch_bounds__(kMiscThreads) void k_gemv_q8w_f32(float* __restrict__ y,
                                                               const uint8_t* __restrict__ W,
                                                               const float* __restrict__ x,
                                                               int rows, int nb, long row_bytes,
                                                               int accumulate) {
    y += (size_t)blockIdx.y * rows;
    x += (size_t)blockIdx.y * nb * 32;
    const long row = misc_row<LPR>();
    const int rl = threadIdx.x % LPR;
    float acc = 0.f;
    if (row < rows) {
        const uint8_t* wr = W + row * row_bytes;
        for (int b = rl; b < nb; b += LPR) {
            const uint8_t* wb = wr + (long)b * 34;
            const float d = h2f(ld2(wb));
            const float4* xb = reinterpret_cast<const float4*>(x + 32 * b);
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t q = ld2x2(wb + 2 + 4 * k);
                const float4 xv = xb[k];
                acc = fmaf(d * (float)(int8_t)(q & 0xff), xv.x, acc);
                acc = fmaf(d * (float)(int8_t)((q >> 8) & 0xff), xv.y, acc);
                acc = fmaf(d * (float)(int8_t)((q >> 16) & 0xff), xv.z, acc);
                acc = fmaf(d * (float)(int8_t)(q >> 24), xv.w, acc);
            }
        }
    }
    acc = lanes_sum<LPR>(acc);
    if (row < rows && rl == 0) y[row] = accumulate ? y[row] + acc : acc;
}

template <int LPR>
__global__ __launch_bounds__(kMiscThreads) void k_gemv_q5_0_f32(float* __restrict__ y,
                                                                const uint8_t* __restrict__ W,
                                                                const float* __restrict__ x,
                                                                int rows, int nb, long row_bytes,
                                                                int accumulate) {
    y += (size_t)blockIdx.y * rows;
    x += (size_t)blockIdx.y * nb * 32;
    const long row = misc_row<LPR>();
    const int rl = threadIdx.x % LPR;
    float acc = 0.f;
    if (row < rows) acc = dot_q5_0_f32<LPR, 32, false>(W + row * row_bytes, x, nb, rl);
    acc = lanes_sum<LPR>(acc);
    if (row < rows && rl == 0) y[row] = accumulate ? y[row] + acc : acc;
}

template <int LPR>
__global__ __launch_bounds__(kMiscThreads) void k_gemv_f16_f32(float* __restrict__ y,
                                                               const uint16_t* __restrict__ W,
                                                               const float* __restrict__ x,
                                                               const float* __restrict__ bias,
                                                               int rows, int cols, int accumulate) {
    y += (size_t)blockIdx.y * rows;
    x += (size_t)blockIdx.y * cols;
    const long row = misc_row<LPR>();
    const int rl = threadIdx.x % LPR;
    float acc = 0.f;
    if (row < rows) acc = dot_f16_f32<LPR, 32>(W + row * (long)cols, x, cols, rl);
    acc = lanes_sum<LPR>(acc);
    if (row < rows && rl == 0) {
        const float v = acc + (bias ? bias[row] : 0.f);
        y[row] = accumulate ? y[row] + v : v;
    }
}

// ---------------------------------------------------------------------------
// A decode stage whose matrices are all Q8_0 / Q5_0 / F16 in one launch:
// RMSNorm(x) * w in every workgroup's prologue (rms_scale<256, 8> and
// q8_block_store: the bits of k_rmsnorm's fp32 and Q8_0 outputs), held in LDS,
// then the rows of up to three matrices (q, k, v) with the row dots above, each
// type on the activation gemv_wt_q8 gives it (llama_model.cpp:767-831: Q8_0
// weights the Q8_0 row, Q5_0 / F16 the fp32 row).  SwiGLU mode (gate, up):
// a workgroup computes R/2 gate rows and the same up rows and writes
// h = swiglu1(gate, up) for them (k_swiglu's arithmetic).  The row dots are
// those of the separate GEMVs; Q5_0 rows take each block's sum of x from the
// prologue (a fixed 8-lane butterfly) where the GEMV sums it alongside the
// products.  With the same lanes per row the Q8_0 and F16 outputs have the
// bits of k_rmsnorm + the GEMV (+ k_swiglu); the lane count is chosen per
// launch (misc_lpr_rows), so the two may differ in fp32 summation order.
// ---------------------------------------------------------------------------
template <int LPR>
__global__ __launch_bounds__(kMiscThreads) void k_misc_norm_stage(MiscStageArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ float red[16];
    constexpr int R = kMiscThreads / LPR;
    __shared__ float gu[R];
    float* xs = reinterpret_cast<float*>(smem);                    // [n/32][36] floats
    uint8_t* xq = smem + (size_t)(a.n / 32) * 36 * sizeof(float);  // [n/32] Q8_0 blocks
    const int n4 = a.n / 4;
    float4 xv[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i4 = threadIdx.x + kMiscThreads * k;
        xv[k] = i4 < n4 ? reinterpret_cast<const float4*>(a.x)[i4] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float s = rms_scale<kMiscThreads, 8>(xv, a.n, a.eps, red);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i4 = threadIdx.x + kMiscThreads * k;
        if (i4 < n4) {
            const float4 v = xv[k];
            const float4 g = reinterpret_cast<const float4*>(a.nw)[i4];
            float4 o;
            o.x = g.x * (v.x * s);
            o.y = g.y * (v.y * s);
            o.z = g.z * (v.z * s);
            o.w = g.w * (v.w * s);
            *reinterpret_cast<float4*>(xs + 36 * (i4 >> 3) + 4 * (i4 & 7)) = o;
            if (a.need_q8) q8_block_store(xq + (size_t)(i4 >> 3) * Q8_0_BYTES, i4 & 7, o);
            // the block's sum of x (Q5_0 rows), into the block's first pad float:
            // the 8 lanes of the block (i4 & 7 == lane & 7) by a fixed butterfly
            float bs = (o.x + o.y) + (o.z + o.w);
            bs += __shfl_xor(bs, 1, 8);
            bs += __shfl_xor(bs, 2, 8);
            bs += __shfl_xor(bs, 4, 8);
            if ((i4 & 7) == 0) xs[36 * (i4 >> 3) + 32] = bs;
        }
    }
    __syncthreads();
    const int li = threadIdx.x / LPR, rl = threadIdx.x % LPR;
    int sg = 0;
    long row;
    if (a.swiglu) {
        sg = li / (R / 2);
        row = (long)blockIdx.x * (R / 2) + li % (R / 2);
    } else {
        row = (long)blockIdx.x * R + li;
        if (a.nseg > 1 && row >= a.rows[0]) {
            row -= a.rows[0];
            sg = 1;
            if (a.nseg > 2 && row >= a.rows[1]) {
                row -= a.rows[1];
                sg = 2;
            }
        }
    }
    // per-segment fields by select (no dynamic indexing of the argument block)
    const uint8_t* W = sg == 0 ? a.W[0] : (sg == 1 ? a.W[1] : a.W[2]);
    const long rb = sg == 0 ? a.rb[0] : (sg == 1 ? a.rb[1] : a.rb[2]);
    const int rows = sg == 0 ? a.rows[0] : (sg == 1 ? a.rows[1] : a.rows[2]);
    const int qt = sg == 0 ? a.qt[0] : (sg == 1 ? a.qt[1] : a.qt[2]);
    float* y = sg == 0 ? a.y[0] : (sg == 1 ? a.y[1] : a.y[2]);
    const bool live = row < rows;
    float acc = 0.f;
    if (live) {
        const uint8_t* wr = W + row * rb;
        if (qt == AXF_TYPE_Q8_0) acc = dot_q8w_q8<LPR>(wr, xq, a.n / 32, rl);
        else if (qt == AXF_TYPE_Q5_0) acc = dot_q5_0_f32<LPR, 36, true>(wr, xs, a.n / 32, rl);
        else acc = dot_f16_f32<LPR, 36>(reinterpret_cast<const uint16_t*>(wr), xs, a.n, rl);
    }
    acc = lanes_sum<LPR>(acc);
    if (!a.swiglu) {
        if (live && rl == 0) y[row] = acc;
        return;
    }
    if (rl == 0) gu[li] = acc;
    __syncthreads();
    if (threadIdx.x < R / 2) {
        const long r = (long)blockIdx.x * (R / 2) + threadIdx.x;
        if (r < a.rows[0]) a.y[0][r] = swiglu1(gu[threadIdx.x], gu[R / 2 + threadIdx.x]);
    }
}

// Embedding row (rows of T tokens when tok_dev lists them): exact dequant.
__global__ __launch_bounds__(256) void k_embed_misc(float* __restrict__ out, int qtype,
                                                    const uint8_t* __restrict__ W,
                                                    const int* __restrict__ tok_dev, int tok,
                                                    int cols, long row_bytes) {
    const int id = tok_dev ? tok_dev[blockIdx.x] : tok;
    const uint8_t* r = W + (long)id * row_bytes;
    float* o = out + (long)blockIdx.x * cols;
    for (int i = threadIdx.x; i < cols; i += 256) {
        float v;
        if (qtype == 1) {  // F16
            v = h2f(ld2(r + 2 * i));
        } else {
            const int b = i >> 5, e = i & 31;
            if (qtype == 8) {  // Q8_0: d * q (q8_0_weight_row_to_f32, :230-243)
                const uint8_t* blk = r + (long)b * 34;
                v = h2f(ld2(blk)) * (float)(int8_t)blk[2 + e];
            } else {  // Q5_0: d * (q5 - 16) (q5_0_row_to_f32, :269-293)
                const uint8_t* blk = r + (long)b * 22;
                const uint32_t qh = ld2x2(blk + 2);
                const uint32_t nib = e < 16 ? (blk[6 + e] & 0x0fu) : (blk[6 + e - 16] >> 4);
                v = h2f(ld2(blk)) * ((float)(nib | (((qh >> e) & 1u) << 4)) - 16.f);
            }
        }
        o[i] = v;
    }
}

int misc_lpr(int units) { return units >= 64 ? 64 : (units >= 32 ? 32 : 16); }

// Lanes per row for a launch of `rows` rows (all tokens): misc_lpr, doubled
// (up to 64) while the launch would have fewer than 256 workgroups; short
// launches then spread each row over more lanes (Qwen2.5-0.5B shape: the
// 896-row o projection 56 -> 224 workgroups, the q|k|v stage 72 -> 288)
static int misc_lpr_rows(int units, long rows) {
    int l = misc_lpr(units);
    while (l < 64 && rows * l < 256L * kMiscThreads) l *= 2;
    return l;
}

// ---------------------------------------------------------------------------
// Batched prefill with fp32 rows (gemm_wt_q8's fallback, llama_model.cpp:876-879,
// runs gemv_wt per token: Q8_0 / Q5_0 / F16 weights on each token's fp32 row).
// The token-grid GEMVs above re-read every weight row once per token; here a
// thread owns one row, dequantises each 32-element block of it once into
// registers and applies it to TT tokens, whose rows every lane of the wave
// reads at the same addresses (scalar-cache loads).  Per token the products are
// summed in k order within each of the workgroup's KS waves (each a
// contiguous range of K), and the KS partials added in wave order through LDS.
// Workgroup = 64 rows x KS waves, grid y = token groups of TT.
// ---------------------------------------------------------------------------
constexpr int kGemmMiscRows = 64;

template <int QT>
__device__ __forceinline__ void misc_block_f32(const uint8_t* __restrict__ wr, int b,
                                               float (&w)[32]) {
    if constexpr (QT == 1) {  // F16: 32 halves, 64 bytes (16-byte aligned rows)
        const uint4* p = reinterpret_cast<const uint4*>(wr + 64 * (long)b);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint4 v = p[k];
            const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                w[8 * k + 2 * j] = h2f(u[j] & 0xffffu);
                w[8 * k + 2 * j + 1] = h2f(u[j] >> 16);
            }
        }
    } else if constexpr (QT == 8) {  // Q8_0: d * q (q8_0_weight_dot_row's weights)
        const uint8_t* wb = wr + (long)b * 34;
        const float d = h2f(ld2(wb));
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t q = ld2x2(wb + 2 + 4 * k);
#pragma unroll
            for (int j = 0; j < 4; j++) w[4 * k + j] = d * (float)(int8_t)((q >> (8 * j)) & 0xffu);
        }
    } else {  // Q5_0: d * (q5 - 16) (q5_0_dot_row's weights)
        const uint8_t* wb = wr + (long)b * 22;
        const float d = h2f(ld2(wb));
        const uint32_t qh = ld2x2(wb + 2);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t qs = ld2x2(wb + 6 + 4 * k);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = 4 * k + j;  // low nibble: element i, high: element i + 16
                w[i] = d * ((float)(((qs >> (8 * j)) & 0x0fu) | (((qh >> i) & 1u) << 4)) - 16.f);
                w[i + 16] = d * ((float)(((qs >> (8 * j + 4)) & 0x0fu) | (((qh >> (i + 16)) & 1u) << 4)) - 16.f);
            }
        }
    }
}

template <int QT, int TT, int KS>
__global__ __launch_bounds__(KS * 64) void k_gemm_misc_f32(
    float* __restrict__ Y, const uint8_t* __restrict__ W, const float* __restrict__ X, int rows,
    int cols, long row_bytes, int T, int accumulate) {
    __shared__ float red[KS][TT][kGemmMiscRows];
    // the wave index as a wave-uniform value, so that the K range and with it
    // every token-row address are uniform: those loads go through the scalar
    // cache (a vector load of one address per lane moved 1 KB per instruction)
    const int lane = threadIdx.x & 63, ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const long row = (long)blockIdx.x * kGemmMiscRows + lane;
    const int t0 = (int)blockIdx.y * TT;
    const uint8_t* wr = W + (row < rows ? row : rows - 1) * row_bytes;  // rows past the end: not stored
    const int nb = cols / 32, nbq = (nb + KS - 1) / KS;
    const int b0 = ks * nbq, b1 = min(nb, b0 + nbq);  // this wave's K range, in blocks
    float acc[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) acc[t] = 0.f;
    for (int b = b0; b < b1; b++) {
        float w[32];
        misc_block_f32<QT>(wr, b, w);
#pragma unroll
        for (int t = 0; t < TT; t++) {
            // token rows past T repeat row T-1 (their sums are not stored)
            const float* xt = X + (size_t)min(t0 + t, T - 1) * cols + 32 * b;
#pragma unroll
            for (int i = 0; i < 32; i++) acc[t] = fmaf(w[i], xt[i], acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < TT; t++) red[ks][t][lane] = acc[t];
    __syncthreads();
    // the KS partial sums of each output, in K order
    for (int o = threadIdx.x; o < TT * kGemmMiscRows; o += KS * 64) {
        const int t = o / kGemmMiscRows, r = o % kGemmMiscRows;
        float v = red[0][t][r];
#pragma unroll
        for (int q = 1; q < KS; q++) v += red[q][t][r];
        const long orow = (long)blockIdx.x * kGemmMiscRows + r;
        if (orow < rows && t0 + t < T) {
            float* y = Y + (size_t)(t0 + t) * rows + orow;
            *y = accumulate ? *y + v : v;
        }
    }
}

// ---------------------------------------------------------------------------
// The same product on the matrix cores (v_mfma_f32_16x16x32_f16):
//   Y[t][o] = sum_b d[o,b] * sum_k c[o,b,k] * x[t, 32b + k]
// with the weight codes c (Q5_0: q5 - 16, Q8_0: q, F16: the stored weight and
// d = 1) exact in fp16.  Token row t is scaled by a power of two 2^E_t
// (max|x_t| * 2^E_t < 2^14) and each scaled value xs (exact) is split as
// hi = fp16(xs), lo = fp16(xs - hi), once per call (k_prep_hl_rows): hi + lo equals xs within ~2^-23
// relative (values below 2^-3 of the row maximum lose low bits of lo only,
// < 2^-37 of the maximum).  Per 32-weight block two MFMAs (A = hi, then lo;
// B = the codes) give the block's sum in fp32, which is scaled by d (Q5_0,
// Q8_0; F16 accumulates in the MFMA), and the result by 2^-E_t.  The sums
// differ from the per-token GEMV's sequential fp32 sums in rounding only.
// Tokens are A's rows and weight rows B's columns: a result lane holds tokens
// 4g..4g+3 of one weight row, so d is the lane's own row's.  A wave owns RTW
// row tiles x TTW token tiles (16 x 16 each); a workgroup 4 waves on
// consecutive row tiles of one token group.
// ---------------------------------------------------------------------------
typedef _Float16 mh8_t __attribute__((ext_vector_type(8)));
typedef _Float16 mh2_t __attribute__((ext_vector_type(2)));
typedef float mf4_t __attribute__((ext_vector_type(4)));
typedef uint32_t mu4_t __attribute__((ext_vector_type(4)));

// wave tile 16 rows x 64 tokens: the Qwen2.5-0.5B-shape 512-token prefill
// 6.60 ms against 6.79 (1 x 8 token tiles), 6.76 (2 x 4), 7.17 (2 x 2),
// 7.32 (1 x 2), 7.83 (4 x 2), 8.98 (2 x 1), 9.59 (4 x 4), 11.0 ms (8 x 2)
constexpr int kMmRTW = 1, kMmTTW = 4, kMmWaves = 4;
constexpr int kMiscMfmaMinT = 16;  // tokens from which the matrix-core form runs

// The A operand of k_gemm_misc_mfma, once per activation: token row t is
// scaled by 2^E_t (max|x_t| * 2^E_t < 2^14, E_t in [-126, 126]) and each group
// of 8 values u = 4b + g (block b, k-group g) stored as 8 fp16 hi then 8 fp16
// lo at xhl[(u * T + t) * 32 bytes]; inv[t] = 2^-E_t.  A workgroup takes 4
// tokens: each wave finds one row's maximum, then the 256 threads convert
// with the token fastest (128 contiguous bytes per group).
__global__ __launch_bounds__(256) void k_prep_hl_rows(const float* __restrict__ X, int cols, int T,
                                                      uint8_t* __restrict__ xhl,
                                                      float* __restrict__ inv) {
    __shared__ float scl[4];
    const int t0 = blockIdx.x * 4, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    {
        const int t = t0 + wave;
        uint32_t m = 0u;  // bits of max |x| (non-negative floats order as integers)
        if (t < T) {
            const float4* xr = reinterpret_cast<const float4*>(X + (size_t)t * cols);
            for (int k = lane; k < cols / 4; k += 64) {
                const float4 v = xr[k];
                m = max(m, max(max(__float_as_uint(v.x) & 0x7fffffffu, __float_as_uint(v.y) & 0x7fffffffu),
                               max(__float_as_uint(v.z) & 0x7fffffffu, __float_as_uint(v.w) & 0x7fffffffu)));
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off, 64));
        // max < 2^(e - 126) for biased exponent e: E = 140 - e keeps it below 2^14
        const int E = max(min(140 - (int)(m >> 23), 126), -126);
        if (lane == 0) {
            scl[wave] = __uint_as_float((uint32_t)(E + 127) << 23);
            if (t < T) inv[t] = __uint_as_float((uint32_t)(127 - E) << 23);
        }
    }
    __syncthreads();
    const int tt = threadIdx.x & 3, t = t0 + tt;
    if (t >= T) return;
    const float sc = scl[tt];
    const float* xr = X + (size_t)t * cols;
    for (int u = threadIdx.x >> 2; u < cols / 8; u += 64) {
        const float4 a = reinterpret_cast<const float4*>(xr + 8 * u)[0];
        const float4 b = reinterpret_cast<const float4*>(xr + 8 * u)[1];
        float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        mh8_t hi, lo;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float xs = v[e] * sc;  // exact: a power-of-two scale
            // hi and lo from this one rounded value (no fusion of the multiply
            // into a mixed-precision conversion for one of them)
            asm volatile("" : "+v"(xs));
            const _Float16 h = (_Float16)xs;
            hi[e] = h;
            lo[e] = (_Float16)(xs - (float)h);
        }
        uint8_t* p = xhl + ((size_t)u * T + t) * 32;
        *reinterpret_cast<mh8_t*>(p) = hi;
        *reinterpret_cast<mh8_t*>(p + 16) = lo;
    }
}

// fp16 pair (1024 + b0 - off, 1024 + b1 - off) of bytes b0, b1 of u picked by sel
__device__ __forceinline__ uint32_t bytes_f16(uint32_t u, uint32_t sel, mh2_t off2) {
    const uint32_t bits = __builtin_amdgcn_perm(0x64646464u, u, sel);
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(mh2_t, bits) + off2);  // exact
}

// The raw words of k-group g of block b of a weight row (loaded one block
// ahead of their use), then the 8 codes as fp16 (B operand) and d.
//   F16: the 16 bytes of the 8 halves;
//   Q8_0: d, two aligned dwords from wb + 8g + sh (sh = wb & 3) and the 16-bit
//         word at wb + 8 + 8g (codes 8g..8g+7 = bytes 2+8g..9+8g);
//   Q5_0: d, 5 aligned dwords from wb + sh and the word at wb + 20 (qh, qs).
// Every byte read lies inside the block.
struct MiscRaw {
    uint32_t w[6];
    uint32_t d;   // fp16 bits of d
    uint32_t sh;  // wb & 3 (0 or 2)
};

template <int QT>
__device__ __forceinline__ void misc_load(const uint8_t* __restrict__ wr, int b, int g, MiscRaw& r) {
    if constexpr (QT == 1) {
        const uint4 v = *reinterpret_cast<const uint4*>(wr + 64 * (long)b + 16 * g);
        r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
    } else {
        const uint8_t* wb = wr + (long)b * (QT == 8 ? 34 : 22);
        r.d = ld2(wb);
        r.sh = (uint32_t)(reinterpret_cast<uintptr_t>(wb) & 3u);
        if constexpr (QT == 8) {
            const uint8_t* wa = wb + 8 * g + r.sh;
            r.w[0] = ld4(wa);
            r.w[1] = ld4(wa + 4);
            r.w[2] = ld2(wb + 8 + 8 * g);
        } else {
            const uint8_t* wa = wb + r.sh;
#pragma unroll
            for (int k = 0; k < 5; k++) r.w[k] = ld4(wa + 4 * k);
            r.w[5] = ld2(wb + 20);
        }
    }
}

template <int QT>
__device__ __forceinline__ mh8_t misc_decode(const MiscRaw& r, int g, float& d) {
    if constexpr (QT == 1) {
        d = 1.f;
        const mu4_t v = {r.w[0], r.w[1], r.w[2], r.w[3]};
        return __builtin_bit_cast(mh8_t, v);
    } else {
        uint32_t q0, q1;  // 8 bytes: Q5_0 q5 in [0, 31], Q8_0 q + 128
        d = h2f(r.d);
        const uint32_t s = 2u - r.sh;
        if constexpr (QT == 8) {
            q0 = alignbyte(r.w[1], r.w[0], s) ^ 0x80808080u;
            q1 = alignbyte(r.w[2], r.w[1], s) ^ 0x80808080u;
        } else {
            const uint32_t qh = alignbyte(r.w[1], r.w[0], s);
            // k-group g: nibbles (low for g < 2) of qs bytes 8(g&1)..8(g&1)+7, qh bits 8g..8g+7
            const int o = 2 * (g & 1);
            const uint32_t qa = alignbyte(o ? r.w[4] : r.w[2], o ? r.w[3] : r.w[1], s);
            const uint32_t qb = alignbyte(o ? r.w[5] : r.w[3], o ? r.w[4] : r.w[2], s);
            const uint32_t ns = 4u * (uint32_t)(g >> 1), hb = qh >> (8 * g);
            q0 = ((qa >> ns) & 0x0f0f0f0fu) | (spread4(hb & 0xfu) << 4);
            q1 = ((qb >> ns) & 0x0f0f0f0fu) | (spread4((hb >> 4) & 0xfu) << 4);
        }
        // fp16 1024 + byte, minus 1024 + 16 (Q5_0) or 1024 + 128 (Q8_0): the code, exact
        const _Float16 o = (_Float16)(QT == 8 ? -1152.f : -1040.f);
        const mh2_t off2 = {o, o};
        const mu4_t v = {bytes_f16(q0, 0x04010400u, off2), bytes_f16(q0, 0x04030402u, off2),
                         bytes_f16(q1, 0x04010400u, off2), bytes_f16(q1, 0x04030402u, off2)};
        return __builtin_bit_cast(mh8_t, v);
    }
}

// KS waves of a workgroup split K (contiguous block ranges, partial tiles added
// in wave order through LDS) and kMmWaves / KS waves take consecutive row
// groups; the block loop loads block b + 1 before computing block b.
template <int QT, int KS>
__global__ __launch_bounds__(kMmWaves * 64) void k_gemm_misc_mfma(
    float* __restrict__ Y, const uint8_t* __restrict__ W, const uint8_t* __restrict__ xhl,
    const float* __restrict__ inv, int rows, int cols, long row_bytes, int T, int accumulate) {
    constexpr int RW = 16 * kMmRTW, TW = 16 * kMmTTW, RG = kMmWaves / KS;
    static_assert(RG * KS == kMmWaves, "waves");
    __shared__ mf4_t part[KS > 1 ? KS - 1 : 1][RG][kMmRTW * kMmTTW][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ks = wave / RG, rg = wave % RG;
    const int col = lane & 15, g = lane >> 4;
    const long row0 = ((long)blockIdx.x * RG + rg) * RW;
    const int t0 = blockIdx.y * TW;
    const uint8_t* wr[kMmRTW];
#pragma unroll
    for (int i = 0; i < kMmRTW; i++)
        wr[i] = W + min(row0 + 16 * i + col, (long)rows - 1) * row_bytes;  // past the end: not stored
    const uint8_t* xr[kMmTTW];  // this lane's token: group u = 4b + g at xr + u*T*32
#pragma unroll
    for (int j = 0; j < kMmTTW; j++) {
        const int t = min(t0 + 16 * j + col, T - 1);  // past T: not stored
        xr[j] = xhl + ((size_t)g * T + t) * 32;
    }
    const mf4_t zero = {0.f, 0.f, 0.f, 0.f};
    mf4_t acc[kMmRTW][kMmTTW];
#pragma unroll
    for (int i = 0; i < kMmRTW; i++)
#pragma unroll
        for (int j = 0; j < kMmTTW; j++) acc[i][j] = zero;
    const int nb = cols / 32, nbq = (nb + KS - 1) / KS;
    const int b0 = ks * nbq, b1 = min(nb, b0 + nbq);
    MiscRaw raw[kMmRTW];
    mh8_t xh[kMmTTW], xl[kMmTTW];
    auto load = [&](int b) {
        const int bb = min(b, nb - 1);  // past the range: a valid block, unused
#pragma unroll
        for (int i = 0; i < kMmRTW; i++) misc_load<QT>(wr[i], bb, g, raw[i]);
#pragma unroll
        for (int j = 0; j < kMmTTW; j++) {
            const uint8_t* p = xr[j] + (size_t)bb * 4 * T * 32;
            xh[j] = *reinterpret_cast<const mh8_t*>(p);
            xl[j] = *reinterpret_cast<const mh8_t*>(p + 16);
        }
    };
    if (b0 < b1) load(b0);
    for (int b = b0; b < b1; b++) {
        mh8_t ah[kMmTTW], al[kMmTTW], bw[kMmRTW];
        float d[kMmRTW];
#pragma unroll
        for (int i = 0; i < kMmRTW; i++) bw[i] = misc_decode<QT>(raw[i], g, d[i]);
#pragma unroll
        for (int j = 0; j < kMmTTW; j++) {
            ah[j] = xh[j];
            al[j] = xl[j];
        }
        if (b + 1 < b1) load(b + 1);  // in flight during this block's products
#pragma unroll
        for (int i = 0; i < kMmRTW; i++)
#pragma unroll
            for (int j = 0; j < kMmTTW; j++) {
                if constexpr (QT == 1) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[j], bw[i], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[j], bw[i], acc[i][j], 0, 0, 0);
                } else {
                    mf4_t c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[j], bw[i], zero, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[j], bw[i], c, 0, 0, 0);
#pragma unroll
                    for (int ii = 0; ii < 4; ii++) acc[i][j][ii] = fmaf(d[i], c[ii], acc[i][j][ii]);
                }
            }
    }
    if constexpr (KS > 1) {
        // partial tiles of K ranges 1..KS-1 through LDS, added to range 0's in order
        if (ks > 0) {
#pragma unroll
            for (int i = 0; i < kMmRTW; i++)
#pragma unroll
                for (int j = 0; j < kMmTTW; j++) part[ks - 1][rg][i * kMmTTW + j][lane] = acc[i][j];
        }
        __syncthreads();
        if (ks > 0) return;
#pragma unroll
        for (int q = 0; q < KS - 1; q++)
#pragma unroll
            for (int i = 0; i < kMmRTW; i++)
#pragma unroll
                for (int j = 0; j < kMmTTW; j++) acc[i][j] += part[q][rg][i * kMmTTW + j][lane];
    }
#pragma unroll
    for (int i = 0; i < kMmRTW; i++) {
        const long o = row0 + 16 * i + col;
#pragma unroll
        for (int j = 0; j < kMmTTW; j++)
#pragma unroll
            for (int ii = 0; ii < 4; ii++) {
                const int t = t0 + 16 * j + 4 * g + ii;
                if (o < rows && t < T) {
                    const float v = acc[i][j][ii] * inv[t];
                    float* y = Y + (size_t)t * rows + o;
                    *y = accumulate ? *y + v : v;
                }
            }
    }
}

template <int TT, int KS>
hipError_t launch_gemm_misc_tt(int qtype, float* Y, const uint8_t* W, const float* X, int rows,
                               int cols, long row_bytes, int T, int accumulate, hipStream_t st) {
    const dim3 grid((unsigned)((rows + kGemmMiscRows - 1) / kGemmMiscRows), (unsigned)((T + TT - 1) / TT));
    const dim3 block(KS * 64);
    if (qtype == 1)
        hipLaunchKernelGGL((k_gemm_misc_f32<1, TT, KS>), grid, block, 0, st, Y, W, X, rows, cols, row_bytes, T, accumulate);
    else if (qtype == 8)
        hipLaunchKernelGGL((k_gemm_misc_f32<8, TT, KS>), grid, block, 0, st, Y, W, X, rows, cols, row_bytes, T, accumulate);
    else
        hipLaunchKernelGGL((k_gemm_misc_f32<6, TT, KS>), grid, block, 0, st, Y, W, X, rows, cols, row_bytes, T, accumulate);
    return hipGetLastError();
}

}  // namespace

// Y (+)= W x^T for T fp32 token rows of cols (Y token-major, rows floats per
// token).  F16 rows must be 16-byte aligned (cols % 32 == 0 makes them so when
// W is); 2-byte-aligned Q8_0 / Q5_0 blocks are read as 16-bit words.
size_t gemm_misc_scratch_bytes(int T, int cols) {
    return (size_t)(T + 3) / 4 * 16 + (size_t)T * cols * 4;  // inv, then hi/lo fp16 rows
}

bool gemm_misc_mfma_applies(int T, const float* X) {
    return T >= kMiscMfmaMinT && (reinterpret_cast<uintptr_t>(X) & 15) == 0;
}

hipError_t launch_gemm_misc_f32(int qtype, float* Y, const void* W, const float* X, int rows,
                                int cols, long row_bytes, int T, int accumulate, hipStream_t st,
                                float* scratch, bool prepared) {
    if (rows <= 0 || T <= 0 || cols <= 0 || cols % 32 || T > 65535 * 16) return hipErrorInvalidValue;
    if (qtype != 1 && qtype != 8 && qtype != 6) return hipErrorInvalidValue;
    if (qtype == 1 && (reinterpret_cast<uintptr_t>(W) & 15)) return hipErrorInvalidValue;
    const auto* w8 = static_cast<const uint8_t*>(W);
    // the matrix cores where there is scratch for the row scales (2 T floats)
    if (scratch && gemm_misc_mfma_applies(T, X)) {
        float* iv = scratch;
        auto* xhl = reinterpret_cast<uint8_t*>(scratch + (T + 3) / 4 * 4);  // 16-byte aligned
        if (!prepared)
            hipLaunchKernelGGL(k_prep_hl_rows, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, st, X,
                               cols, T, xhl, iv);
        // K split over the workgroup's waves where the row groups x token groups
        // leave fewer than 2048 workgroups (K ranges of at least 4 blocks)
        const long tg = (T + 16 * kMmTTW - 1) / (16 * kMmTTW), nb = cols / 32;
        auto wgs = [&](int ks) { return (rows + 16L * kMmRTW * (kMmWaves / ks) - 1) / (16L * kMmRTW * (kMmWaves / ks)) * tg; };
        int ks = 1;
        while (ks < kMmWaves && wgs(ks) < 2048 && nb >= 8L * ks) ks *= 2;
        const dim3 grid((unsigned)(wgs(ks) / tg), (unsigned)tg);
#define AXF_MM(QT_, KS_) \
    hipLaunchKernelGGL((k_gemm_misc_mfma<QT_, KS_>), grid, dim3(kMmWaves * 64), 0, st, Y, w8, xhl, iv, rows, cols, row_bytes, T, accumulate)
#define AXF_MM_KS(QT_) \
    do { if (ks == 4) AXF_MM(QT_, 4); else if (ks == 2) AXF_MM(QT_, 2); else AXF_MM(QT_, 1); } while (0)
        if (qtype == 1) AXF_MM_KS(1);
        else if (qtype == 8) AXF_MM_KS(8);
        else AXF_MM_KS(6);
#undef AXF_MM_KS
#undef AXF_MM
        return hipGetLastError();
    }
    // waves = row groups x token groups x K ranges: 32 tokens per group and 4
    // K ranges where that gives 4096 waves (4 per SIMD) or K is under 16
    // blocks, else 16 tokens with 4, then 8 K ranges (a wave past the last
    // block adds zeros)
    const long rg = (rows + kGemmMiscRows - 1) / kGemmMiscRows;
    const int nb = cols / 32;
    if (rg * ((T + 31) / 32) * 4 >= 4096 || nb < 16)
        return launch_gemm_misc_tt<32, 4>(qtype, Y, w8, X, rows, cols, row_bytes, T, accumulate, st);
    if (rg * ((T + 15) / 16) * 4 >= 4096)
        return launch_gemm_misc_tt<16, 4>(qtype, Y, w8, X, rows, cols, row_bytes, T, accumulate, st);
    return launch_gemm_misc_tt<16, 8>(qtype, Y, w8, X, rows, cols, row_bytes, T, accumulate, st);
}

#define AXF_MISC_LAUNCH(KERNEL, LPR_, ROWS, ...)                                           \
    do {                                                                                   \
        const dim3 grid_((unsigned)(((long)(ROWS) + (kMiscThreads / LPR_) - 1) /           \
                                    (kMiscThreads / LPR_)), (unsigned)T);                 \
        hipLaunchKernelGGL((KERNEL<LPR_>), grid_, dim3(kMiscThreads), 0, st, __VA_ARGS__); \
    } while (0)

#define AXF_MISC_DISPATCH(KERNEL, UNITS, ROWS, ...)                                        \
    do {                                                                                   \
        const int l_ = misc_lpr_rows(UNITS, (long)(ROWS) * T);                            \
        if (l_ == 64) AXF_MISC_LAUNCH(KERNEL, 64, ROWS, __VA_ARGS__);                      \
        else if (l_ == 32) AXF_MISC_LAUNCH(KERNEL, 32, ROWS, __VA_ARGS__);                 \
        else AXF_MISC_LAUNCH(KERNEL, 16, ROWS, __VA_ARGS__);                               \
    } while (0)

hipError_t launch_gemv_q8w_q8(float* y, const void* W, const void* xq8, int rows, int nb,
                              long row_bytes, int accumulate, hipStream_t st, int T) {
    if (T <= 0 || T > 65535) return hipErrorInvalidValue;
    AXF_MISC_DISPATCH(k_gemv_q8w_q8, nb, rows, y, static_cast<const uint8_t*>(W),
                      static_cast<const uint8_t*>(xq8), rows, nb, row_bytes, accumulate);
    return hipGetLastError();
}

hipError_t launch_gemv_q8w_f32(float* y, const void* W, const float* x, int rows, int nb,
                               long row_bytes, hipStream_t st, int accumulate, int T) {
    if (T <= 0 || T > 65535) return hipErrorInvalidValue;
    AXF_MISC_DISPATCH(k_gemv_q8w_f32, nb, rows, y, static_cast<const uint8_t*>(W), x, rows, nb,
                      row_bytes, accumulate);
    return hipGetLastError();
}

hipError_t launch_gemv_q5_0_f32(float* y, const void* W, const float* x, int rows, int nb,
                                long row_bytes, hipStream_t st, int accumulate, int T) {
    if (T <= 0 || T > 65535) return hipErrorInvalidValue;
    AXF_MISC_DISPATCH(k_gemv_q5_0_f32, nb, rows, y, static_cast<const uint8_t*>(W), x, rows, nb,
                      row_bytes, accumulate);
    return hipGetLastError();
}

hipError_t launch_gemv_f16_f32(float* y, const void* W, const float* x, const float* bias,
                               int rows, int cols, hipStream_t st, int accumulate, int T) {
    if (T <= 0 || T > 65535) return hipErrorInvalidValue;
    AXF_MISC_DISPATCH(k_gemv_f16_f32, cols / 8, rows, y, static_cast<const uint16_t*>(W), x, bias,
                      rows, cols, accumulate);
    return hipGetLastError();
}

static int misc_mat_lpr(int qtype, int n) { return misc_lpr(qtype == AXF_TYPE_F16 ? n / 8 : n / 32); }

bool misc_norm_stage_ok(const MiscMat* mats, int nmat, int n) {
    if (nmat < 1 || nmat > 3 || n <= 0 || n % 32 || n > 8192) return false;
    for (int i = 0; i < nmat; i++) {
        const int qt = mats[i].qtype;
        if (qt != AXF_TYPE_Q8_0 && qt != AXF_TYPE_Q5_0 && qt != AXF_TYPE_F16) return false;
        if (qt == AXF_TYPE_F16 && (reinterpret_cast<uintptr_t>(mats[i].W) & 15)) return false;
        if (mats[i].rows <= 0 || misc_mat_lpr(qt, n) != misc_mat_lpr(mats[0].qtype, n)) return false;
    }
    return true;
}

hipError_t launch_misc_norm_stage(const MiscMat* mats, int nmat, bool swiglu, const float* x,
                                  const float* nw, float eps, int n, hipStream_t st) {
    if (!misc_norm_stage_ok(mats, nmat, n) || (swiglu && (nmat != 2 || mats[0].rows != mats[1].rows)))
        return hipErrorInvalidValue;
    MiscStageArgs a{};
    a.x = x;
    a.nw = nw;
    a.eps = eps;
    a.n = n;
    a.nseg = nmat;
    a.swiglu = swiglu ? 1 : 0;
    long total = 0;
    for (int i = 0; i < 3; i++) {
        const MiscMat& mm = mats[i < nmat ? i : 0];
        a.W[i] = static_cast<const uint8_t*>(mm.W);
        a.rb[i] = mm.row_bytes;
        a.rows[i] = i < nmat ? mm.rows : 0;
        a.qt[i] = mm.qtype;
        a.y[i] = mm.y;
        if (i < nmat) {
            total += mm.rows;
            a.need_q8 |= mm.qtype == AXF_TYPE_Q8_0;
        }
    }
    const int lpr = misc_lpr_rows(mats[0].qtype == AXF_TYPE_F16 ? n / 8 : n / 32,
                                  swiglu ? 2L * mats[0].rows : total);
    const int R = kMiscThreads / lpr;
    const long wgs = swiglu ? (mats[0].rows + R / 2 - 1) / (R / 2) : (total + R - 1) / R;
    const size_t lds = (size_t)(n / 32) * (36 * sizeof(float) + (a.need_q8 ? Q8_0_BYTES : 0));
    if (lpr == 64)
        hipLaunchKernelGGL(k_misc_norm_stage<64>, dim3((unsigned)wgs), dim3(kMiscThreads), lds, st, a);
    else if (lpr == 32)
        hipLaunchKernelGGL(k_misc_norm_stage<32>, dim3((unsigned)wgs), dim3(kMiscThreads), lds, st, a);
    else
        hipLaunchKernelGGL(k_misc_norm_stage<16>, dim3((unsigned)wgs), dim3(kMiscThreads), lds, st, a);
    return hipGetLastError();
}

hipError_t launch_embed_misc(int qtype, float* out, const void* W, const int* tok_dev, int tok,
                             int T, int cols, long row_bytes, hipStream_t st) {
    hipLaunchKernelGGL(k_embed_misc, dim3((unsigned)T), dim3(256), 0, st, out, qtype,
                       static_cast<const uint8_t*>(W), tok_dev, tok, cols, row_bytes);
    return hipGetLastError();
}

}  // namespace axf
