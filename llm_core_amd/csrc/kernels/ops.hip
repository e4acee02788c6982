// ops.hip — dequantisation, Q8_0 quantisation and the decode-step operations
// around the GEMVs (RMSNorm, RoPE + KV store, single-token attention, SwiGLU,
// embedding row, argmax) for gfx950.
//
// Device-side position: kernels that run inside a captured decode graph read
// the position from device memory (pos_dev != nullptr) so one graph serves
// every step; otherwise the immediate `pos` is used.
#include "common.hpp"

namespace axf {

__device__ __forceinline__ int read_pos(const int* pos_dev, int pos) {
    return pos_dev ? *pos_dev : pos;
}

// ---------------------------------------------------------------------------
// Dequantisation (bit-exact with the reference's scalar dequant)
// ---------------------------------------------------------------------------

// Q4_K: out = fma(d*sc, q, -(dmin*m)); one thread per 4 qs bytes (8 outputs).
__global__ void k_dequant_q4k(float* __restrict__ out, const uint8_t* __restrict__ W,
                              long nblocks) {
    const long n = nblocks * 32;
    for (long t = (long)blockIdx.x * blockDim.x + threadIdx.x; t < n;
         t += (long)gridDim.x * blockDim.x) {
        const long b = t >> 5;
        const int k = (int)(t & 31), c = k >> 3, l0 = (k & 7) * 4;
        const uint8_t* blk = W + b * Q4K_BYTES;
        const uint4 h = ld16(blk);
        const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        q4k_scales(h.y, h.z, h.w, c, sc0, m0, sc1, m1);
        const float d1 = d * (float)sc0, mf1 = dmin * (float)m0;
        const float d2 = d * (float)sc1, mf2 = dmin * (float)m1;
        const uint32_t q = ld4(blk + 16 + 32 * c + l0);
        float* o = out + b * QK_K + 64 * c + l0;
        float4 lo, hi;
        lo.x = fmaf(d1, (float)(q & 0xfu), -mf1);
        lo.y = fmaf(d1, (float)((q >> 8) & 0xfu), -mf1);
        lo.z = fmaf(d1, (float)((q >> 16) & 0xfu), -mf1);
        lo.w = fmaf(d1, (float)((q >> 24) & 0xfu), -mf1);
        hi.x = fmaf(d2, (float)((q >> 4) & 0xfu), -mf2);
        hi.y = fmaf(d2, (float)((q >> 12) & 0xfu), -mf2);
        hi.z = fmaf(d2, (float)((q >> 20) & 0xfu), -mf2);
        hi.w = fmaf(d2, (float)((q >> 28) & 0xfu), -mf2);
        *reinterpret_cast<float4*>(o) = lo;
        *reinterpret_cast<float4*>(o + 32) = hi;
    }
}

// Q6_K: out = (d*sc)*(q-32); one thread per (block, half, 4 consecutive l).
__global__ void k_dequant_q6k(float* __restrict__ out, const uint8_t* __restrict__ W,
                              long nblocks) {
    const long n = nblocks * 16;
    for (long t = (long)blockIdx.x * blockDim.x + threadIdx.x; t < n;
         t += (long)gridDim.x * blockDim.x) {
        const long b = t >> 4;
        const int k = (int)(t & 15), half = k >> 3, l0 = (k & 7) * 4;
        const uint8_t* blk = W + b * Q6K_BYTES;
        const float d = h2f(ld2(blk + 208));
        const uint8_t* ql = blk + 64 * half;
        const uint8_t* qh = blk + 128 + 32 * half;
        const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192 + 8 * half);
        float* y = out + b * QK_K + 128 * half;
        const int is = l0 / 16;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int l = l0 + j;
            const int q1 = ((ql[l] & 0x0f) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = ((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l + 0] = (d * (float)sc[is + 0]) * (float)q1;
            y[l + 32] = (d * (float)sc[is + 2]) * (float)q2;
            y[l + 64] = (d * (float)sc[is + 4]) * (float)q3;
            y[l + 96] = (d * (float)sc[is + 6]) * (float)q4;
        }
    }
}

// ---------------------------------------------------------------------------
// Q8_0 quantisation: 8 lanes per 32-element block, 4 elements per lane.
// d = amax/127, id = 127/amax (0 when amax == 0), q = rne(x*id) saturated.
// ---------------------------------------------------------------------------
__global__ void k_quantize_q8_0(uint8_t* __restrict__ y, const float* __restrict__ x, int n) {
    const int nthreads = n / 4;  // n % 32 == 0
    for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < nthreads; t += gridDim.x * blockDim.x) {
        // all 8 lanes of a block are in the same iteration: nthreads % 8 == 0 and
        // the grid stride is a multiple of 8
        const float4 v = reinterpret_cast<const float4*>(x)[t];
        q8_block_store(y + (size_t)(t >> 3) * Q8_0_BYTES, t & 7, v);
    }
}

// ---------------------------------------------------------------------------
// RMSNorm (+ optional Q8_0 of the result), one workgroup of 1024 threads:
// y = w*(x*s), s = 1/sqrt(sum(x^2)/n + eps) (rms_norm_out, llama_model.cpp:396-419).
// The scale is rms_scale's, the same bits the GEMV prologues that fuse
// this norm compute (the extra zero float4s of n <= 8192 add exact zeros).
// n <= 32768.
// ---------------------------------------------------------------------------
constexpr int kNormThreads = 1024;

__global__ __launch_bounds__(kNormThreads) void k_rmsnorm(float* __restrict__ y,
                                                          uint8_t* __restrict__ yq8,
                                                          const float* __restrict__ x,
                                                          const float* __restrict__ w, int n,
                                                          float eps) {
    __shared__ float red[16];
    // row blockIdx.x of a [rows][n] batch
    x += (size_t)blockIdx.x * n;
    if (y) y += (size_t)blockIdx.x * n;
    if (yq8) yq8 += (size_t)blockIdx.x * (n / 32) * Q8_0_BYTES;
    const int n4 = n / 4;
    float4 xv[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i4 = threadIdx.x + kNormThreads * k;
        xv[k] = i4 < n4 ? reinterpret_cast<const float4*>(x)[i4] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float s = rms_scale<kNormThreads, 8>(xv, n, eps, red);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i4 = threadIdx.x + kNormThreads * k;
        if (i4 < n4) {
            const float4 v = xv[k];
            const float4 g = reinterpret_cast<const float4*>(w)[i4];
            float4 o;
            o.x = g.x * (v.x * s);
            o.y = g.y * (v.y * s);
            o.z = g.z * (v.z * s);
            o.w = g.w * (v.w * s);
            if (y) reinterpret_cast<float4*>(y)[i4] = o;
            if (yq8) q8_block_store(yq8 + (size_t)(i4 >> 3) * Q8_0_BYTES, i4 & 7, o);
        }
    }
}

// The row RMSNorm of k_rmsnorm (same arithmetic, same Q8_0 blocks) that also
// writes the prefill GEMMs' activation re-layout in the same pass, as
// k_gemm_prep16 would from the blocks: for row t and Q8_0 block kb,
//   xh[kb][g][Tp][8]  fp16 copies of values 8g..8g+7,
//   dx2, gx2          d and d * (sum of the 32 int8) at the 32-token-group
//                     index of the fp16 Q4_K GEMM,
//   dx4               d at the 64-token-group index of the fp16 Q6_K GEMM.
// The grid covers Tp rows: rows T..Tp-1 write zeros there (and nothing else).
// NT threads per row, n <= 32 * NT (rms_scale's partial sums do not depend on NT).
template <int NT>
__global__ __launch_bounds__(NT) void k_rmsnorm_prep(
    float* __restrict__ y, uint8_t* __restrict__ yq8, const float* __restrict__ x,
    const float* __restrict__ w, int n, float eps, int T, int Tp, uint8_t* __restrict__ xh,
    float* __restrict__ dx2, float* __restrict__ gx2, float* __restrict__ dx4) {
    __shared__ float red[16];
    // workgroup L runs on XCD L % 8: rows (L % 8) * Tp/8 ... on one XCD, so the
    // 8 rows whose 16-byte xh pieces share a 128-byte line meet in one L2
    const int L = blockIdx.x, t = (L & 7) * (Tp >> 3) + (L >> 3), n4 = n / 4;
    auto idx = [&](int kb, int ttw) {  // k_gemm_prep16's dx index for 16*ttw-token groups
        const int tw = 16 * ttw;
        return (((size_t)kb * (Tp / tw) + t / tw) * 16 + (t & 15)) * ttw + ((t >> 4) % ttw);
    };
    if (t >= T) {  // padding rows: zero activations
        for (int i4 = threadIdx.x; i4 < n4; i4 += NT) {
            const int kb = i4 >> 3, sub = i4 & 7;
            *reinterpret_cast<uint2*>(xh + (((size_t)kb * 4 + (sub >> 1)) * Tp + t) * 16 +
                                      (sub & 1) * 8) = make_uint2(0u, 0u);
            if (sub == 0) {
                dx2[idx(kb, 2)] = 0.f;
                gx2[idx(kb, 2)] = 0.f;
                dx4[idx(kb, 4)] = 0.f;
            }
        }
        return;  // the whole workgroup (before any barrier)
    }
    x += (size_t)t * n;
    if (y) y += (size_t)t * n;
    yq8 += (size_t)t * (n / 32) * Q8_0_BYTES;
    float4 xv[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i4 = threadIdx.x + NT * k;
        xv[k] = i4 < n4 ? reinterpret_cast<const float4*>(x)[i4] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float s = rms_scale<NT, 8>(xv, n, eps, red);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i4 = threadIdx.x + NT * k;
        if (i4 < n4) {  // the 8 lanes of a block share it
            const float4 v = xv[k];
            const float4 g = reinterpret_cast<const float4*>(w)[i4];
            float4 o;
            o.x = g.x * (v.x * s);
            o.y = g.y * (v.y * s);
            o.z = g.z * (v.z * s);
            o.w = g.w * (v.w * s);
            if (y) reinterpret_cast<float4*>(y)[i4] = o;
            const int kb = i4 >> 3, sub = i4 & 7;
            float d;
            const uint32_t p = q8_quant4(o, d);  // q8_block_store's block
            uint8_t* blk = yq8 + (size_t)kb * Q8_0_BYTES;
            *reinterpret_cast<uint32_t*>(blk + 4 + 4 * sub) = p;
            if (sub == 0) *reinterpret_cast<float*>(blk) = d;
            // fp16 of the 4 int8, then d and d * sum for the block (8 lanes)
            _Float16 hv[4];
#pragma unroll
            for (int e = 0; e < 4; e++) hv[e] = (_Float16)(float)(int8_t)(p >> (8 * e));
            *reinterpret_cast<uint2*>(xh + (((size_t)kb * 4 + (sub >> 1)) * Tp + t) * 16 +
                                      (sub & 1) * 8) = *reinterpret_cast<const uint2*>(hv);
            int sum = dot4((int)p, 0x01010101, 0);
            sum += __shfl_xor(sum, 1, 8);
            sum += __shfl_xor(sum, 2, 8);
            sum += __shfl_xor(sum, 4, 8);
            if (sub == 0) {
                dx2[idx(kb, 2)] = d;
                gx2[idx(kb, 2)] = d * (float)sum;
                dx4[idx(kb, 4)] = d;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// RoPE (rotate-half pairs (i, i+hd/2)) with the host-built cos/sin table:
//   a = fma(x0, c, -(x1*s)),  b = fma(x0, s, x1*c)
// k_rope: dst may alias src.  k_rope_qkv: q in place, k -> kcache row pos,
// v copied to vcache row pos.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void rope_pair(const float* src, float* dst, int i, int half,
                                          const float* cr, const float* sr) {
    const float x0 = src[i], x1 = src[i + half];
    const float c = cr[i], s = sr[i];
    const float a = fmaf(x0, c, -(x1 * s));
    const float b = fmaf(x0, s, x1 * c);
    dst[i] = a;
    dst[i + half] = b;
}

__global__ void k_rope(float* dst, const float* src, const int* pos_dev, int pos, int n_heads,
                       int hd, const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
    const int half = hd / 2;
    const int p = read_pos(pos_dev, pos);
    const float* cr = cos_t + (size_t)p * half;
    const float* sr = sin_t + (size_t)p * half;
    for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < n_heads * half;
         t += gridDim.x * blockDim.x) {
        const int h = t / half, i = t % half;
        rope_pair(src + (size_t)h * hd, dst + (size_t)h * hd, i, half, cr, sr);
    }
}

__global__ void k_rope_qkv(float* q, const float* __restrict__ k, const float* __restrict__ v,
                           float* __restrict__ kcache, float* __restrict__ vcache,
                           const int* pos_dev, int pos, int n_heads, int n_kv_heads, int hd,
                           const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
    const int half = hd / 2;
    const int p = read_pos(pos_dev, pos);
    const size_t kv_embd = (size_t)n_kv_heads * hd;
    const float* cr = cos_t + (size_t)p * half;
    const float* sr = sin_t + (size_t)p * half;
    float* krow = kcache + (size_t)p * kv_embd;
    float* vrow = vcache + (size_t)p * kv_embd;
    const int nq = n_heads * half, nk = n_kv_heads * half;
    for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < nq + nk + (int)kv_embd;
         t += gridDim.x * blockDim.x) {
        if (t < nq) {
            const int h = t / half, i = t % half;
            rope_pair(q + (size_t)h * hd, q + (size_t)h * hd, i, half, cr, sr);
        } else if (t < nq + nk) {
            const int u = t - nq, h = u / half, i = u % half;
            rope_pair(k + (size_t)h * hd, krow + (size_t)h * hd, i, half, cr, sr);
        } else {
            const int u = t - nq - nk;
            vrow[u] = v[u];
        }
    }
}

// ---------------------------------------------------------------------------
// SwiGLU (swiglu1 in common.hpp).  Optional Q8_0 of the result.  gate/up may
// be separate buffers or halves of one buffer.
// ---------------------------------------------------------------------------
__global__ void k_swiglu(float* __restrict__ out, uint8_t* __restrict__ outq8,
                         const float* __restrict__ gate, const float* __restrict__ up, int n) {
    const int nthreads = n / 4;
    for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < nthreads; t += gridDim.x * blockDim.x) {
        const float4 g = reinterpret_cast<const float4*>(gate)[t];
        const float4 u = reinterpret_cast<const float4*>(up)[t];
        float4 o;
        o.x = swiglu1(g.x, u.x);
        o.y = swiglu1(g.y, u.y);
        o.z = swiglu1(g.z, u.z);
        o.w = swiglu1(g.w, u.w);
        if (out) reinterpret_cast<float4*>(out)[t] = o;
        if (outq8) q8_block_store(outq8 + (size_t)(t >> 3) * Q8_0_BYTES, t & 7, o);
    }
}

// ---------------------------------------------------------------------------
// K/V of T tokens into the cache (batched prefill): row t at position pos0+t,
//   kcache[pos] = RoPE(k_t + bk),  vcache[pos] = v_t + bv
// (add_bias_rows then rope_and_store_k / the V copy of llama_forward_batch,
// src/models/llama_model.cpp:1380-1406).  k_t = k + t*k_ld, v_t = v + t*v_ld.
// ---------------------------------------------------------------------------
__global__ void k_rope_kv_rows(const float* __restrict__ k, int k_ld, const float* __restrict__ v,
                               int v_ld, const float* __restrict__ bk,
                               const float* __restrict__ bv, float* __restrict__ kcache,
                               float* __restrict__ vcache, int pos0, int n_kv_heads, int hd,
                               const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
    const int half = hd / 2;
    const int t = blockIdx.y, p = pos0 + t;
    const size_t kv_embd = (size_t)n_kv_heads * hd;
    const float* cr = cos_t + (size_t)p * half;
    const float* sr = sin_t + (size_t)p * half;
    const float* kr = k + (size_t)t * k_ld;
    const float* vr = v + (size_t)t * v_ld;
    float* krow = kcache + (size_t)p * kv_embd;
    float* vrow = vcache + (size_t)p * kv_embd;
    const int nk = n_kv_heads * half;
    for (int u = blockIdx.x * blockDim.x + threadIdx.x; u < nk + (int)kv_embd;
         u += gridDim.x * blockDim.x) {
        if (u < nk) {
            const int h = u / half, i = u % half;
            const size_t e0 = (size_t)h * hd + i, e1 = e0 + half;
            const float x0 = bk ? kr[e0] + bk[e0] : kr[e0];
            const float x1 = bk ? kr[e1] + bk[e1] : kr[e1];
            const float c = cr[i], s = sr[i];
            krow[e0] = fmaf(x0, c, -(x1 * s));
            krow[e1] = fmaf(x0, s, x1 * c);
        } else {
            const int e = u - nk;
            vrow[e] = bv ? vr[e] + bv[e] : vr[e];
        }
    }
}

// The same, four consecutive elements per thread (float4 loads and stores;
// hd % 8 == 0, 16-byte aligned rows, caches, biases and RoPE tables): the
// same operations on each element.
__global__ void k_rope_kv_rows4(const float* __restrict__ k, int k_ld, const float* __restrict__ v,
                                int v_ld, const float* __restrict__ bk,
                                const float* __restrict__ bv, float* __restrict__ kcache,
                                float* __restrict__ vcache, int pos0, int n_kv_heads, int hd,
                                const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
    const int half = hd / 2;
    const int t = blockIdx.y, p = pos0 + t;
    const size_t kv_embd = (size_t)n_kv_heads * hd;
    const float* cr = cos_t + (size_t)p * half;
    const float* sr = sin_t + (size_t)p * half;
    const float* kr = k + (size_t)t * k_ld;
    const float* vr = v + (size_t)t * v_ld;
    float* krow = kcache + (size_t)p * kv_embd;
    float* vrow = vcache + (size_t)p * kv_embd;
    const int nk4 = n_kv_heads * half / 4, nv4 = (int)(kv_embd / 4);
    auto ld = [](const float* a, size_t e) { return *reinterpret_cast<const float4*>(a + e); };
    for (int u = blockIdx.x * blockDim.x + threadIdx.x; u < nk4 + nv4; u += gridDim.x * blockDim.x) {
        if (u < nk4) {
            const int h = (4 * u) / half, i = (4 * u) % half;
            const size_t e0 = (size_t)h * hd + i, e1 = e0 + half;
            float4 x0 = ld(kr, e0), x1 = ld(kr, e1);
            if (bk) {
                const float4 b0 = ld(bk, e0), b1 = ld(bk, e1);
                x0 = make_float4(x0.x + b0.x, x0.y + b0.y, x0.z + b0.z, x0.w + b0.w);
                x1 = make_float4(x1.x + b1.x, x1.y + b1.y, x1.z + b1.z, x1.w + b1.w);
            }
            const float4 c = ld(cr, i), sn = ld(sr, i);
            *reinterpret_cast<float4*>(krow + e0) =
                make_float4(fmaf(x0.x, c.x, -(x1.x * sn.x)), fmaf(x0.y, c.y, -(x1.y * sn.y)),
                            fmaf(x0.z, c.z, -(x1.z * sn.z)), fmaf(x0.w, c.w, -(x1.w * sn.w)));
            *reinterpret_cast<float4*>(krow + e1) =
                make_float4(fmaf(x0.x, sn.x, x1.x * c.x), fmaf(x0.y, sn.y, x1.y * c.y),
                            fmaf(x0.z, sn.z, x1.z * c.z), fmaf(x0.w, sn.w, x1.w * c.w));
        } else {
            const size_t e = (size_t)(u - nk4) * 4;
            float4 x = ld(vr, e);
            if (bv) {
                const float4 b = ld(bv, e);
                x = make_float4(x.x + b.x, x.y + b.y, x.z + b.z, x.w + b.w);
            }
            *reinterpret_cast<float4*>(vrow + e) = x;
        }
    }
}

// SwiGLU of T rows whose gate and up halves are interleaved by row blocks of B
// ([gate B][up B] ... per row of 2*n), into Q8_0 blocks of the [T][n] result.
__global__ void k_swiglu_gu(uint8_t* __restrict__ outq8, float* __restrict__ out,
                            const float* __restrict__ gu, int T, int n, int B) {
    const int n4 = n / 4;
    for (long q = (long)blockIdx.x * blockDim.x + threadIdx.x; q < (long)T * n4;
         q += (long)gridDim.x * blockDim.x) {
        const long t = q / n4;
        const int f = (int)(q - t * n4) * 4;
        const int j = f / B, r = f - j * B;
        const float* row = gu + (size_t)t * 2 * n + (size_t)2 * j * B + r;
        const float4 g = *reinterpret_cast<const float4*>(row);
        const float4 u = *reinterpret_cast<const float4*>(row + B);
        float4 o;
        o.x = swiglu1(g.x, u.x);
        o.y = swiglu1(g.y, u.y);
        o.z = swiglu1(g.z, u.z);
        o.w = swiglu1(g.w, u.w);
        if (out) reinterpret_cast<float4*>(out)[q] = o;  // [T][n] fp32 rows
        q8_block_store(outq8 + (size_t)(q >> 3) * Q8_0_BYTES, (int)(q & 7), o);
    }
}

// ---------------------------------------------------------------------------
// Embedding row (token id from device memory or immediate): dequantise row
// `tok` of a Q4_K / Q6_K matrix with `nb` blocks per row.
// ---------------------------------------------------------------------------
__global__ void k_embed_q4k(float* __restrict__ out, const uint8_t* __restrict__ W,
                            const int* tok_dev, int tok, int nb, long row_bytes) {
    // row blockIdx.x: token tok_dev[blockIdx.x] (or tok) into out + blockIdx.x * nb * 256
    const int id = tok_dev ? tok_dev[blockIdx.x] : tok;
    out += (size_t)blockIdx.x * nb * QK_K;
    const uint8_t* row = W + (long)id * row_bytes;
    for (int t = threadIdx.x; t < nb * 32; t += blockDim.x) {
        const int b = t >> 5, k = t & 31, c = k >> 3, l0 = (k & 7) * 4;
        const uint8_t* blk = row + (long)b * Q4K_BYTES;
        const uint4 h = ld16(blk);
        const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        q4k_scales(h.y, h.z, h.w, c, sc0, m0, sc1, m1);
        const float d1 = d * (float)sc0, mf1 = dmin * (float)m0;
        const float d2 = d * (float)sc1, mf2 = dmin * (float)m1;
        const uint32_t q = ld4(blk + 16 + 32 * c + l0);
        float* o = out + b * QK_K + 64 * c + l0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            o[e] = fmaf(d1, (float)((q >> (8 * e)) & 0xfu), -mf1);
            o[32 + e] = fmaf(d2, (float)((q >> (8 * e + 4)) & 0xfu), -mf2);
        }
    }
}

__global__ void k_embed_q6k(float* __restrict__ out, const uint8_t* __restrict__ W,
                            const int* tok_dev, int tok, int nb, long row_bytes) {
    // row blockIdx.x: token tok_dev[blockIdx.x] (or tok) into out + blockIdx.x * nb * 256
    const int id = tok_dev ? tok_dev[blockIdx.x] : tok;
    out += (size_t)blockIdx.x * nb * QK_K;
    const uint8_t* row = W + (long)id * row_bytes;
    for (int t = threadIdx.x; t < nb * 128; t += blockDim.x) {
        const int b = t >> 7, k = t & 127, half = k >> 6, l = k & 31, s = (k >> 5) & 1;
        const uint8_t* blk = row + (long)b * Q6K_BYTES;
        const float d = h2f(ld2(blk + 208));
        const uint8_t* ql = blk + 64 * half;
        const uint8_t* qh = blk + 128 + 32 * half;
        const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192 + 8 * half);
        const int is = l / 16;
        float* y = out + b * QK_K + 128 * half;
        if (s == 0) {
            const int q1 = ((ql[l] & 0x0f) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            y[l] = (d * (float)sc[is]) * (float)q1;
            y[l + 64] = (d * (float)sc[is + 4]) * (float)q3;
        } else {
            const int q2 = ((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l + 32] = (d * (float)sc[is + 2]) * (float)q2;
            y[l + 96] = (d * (float)sc[is + 6]) * (float)q4;
        }
    }
}

// ---------------------------------------------------------------------------
// argmax (first index of the maximum, std::max_element semantics), two stages.
// ---------------------------------------------------------------------------
constexpr int kArgThreads = 256;

__device__ __forceinline__ void argmax_merge(float& v, int& i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

__device__ __forceinline__ void block_argmax(float& v, int& i) {
    __shared__ float sv[kArgThreads / 64];
    __shared__ int si[kArgThreads / 64];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float v2 = __shfl_xor(v, off, 64);
        const int i2 = __shfl_xor(i, off, 64);
        argmax_merge(v, i, v2, i2);
    }
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) {
        sv[w] = v;
        si[w] = i;
    }
    __syncthreads();
    v = sv[0];
    i = si[0];
#pragma unroll
    for (int k = 1; k < kArgThreads / 64; k++) argmax_merge(v, i, sv[k], si[k]);
}

__global__ __launch_bounds__(kArgThreads) void k_argmax_partial(float* __restrict__ pv,
                                                                int* __restrict__ pi,
                                                                const float* __restrict__ x,
                                                                int n) {
    float v = -INFINITY;
    int i = 0x7fffffff;
    for (int t = blockIdx.x * kArgThreads + threadIdx.x; t < n; t += gridDim.x * kArgThreads)
        argmax_merge(v, i, x[t], t);
    block_argmax(v, i);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = v;
        pi[blockIdx.x] = i;
    }
}

// Final stage; also appends the token to `tokens[*step]` and advances the
// device-side position/step counters when they are given (decode graph).
__global__ __launch_bounds__(kArgThreads) void k_argmax_final(int* __restrict__ out,
                                                              const float* __restrict__ pv,
                                                              const int* __restrict__ pi,
                                                              int nparts, int* tokens,
                                                              int* step, int* pos) {
    float v = -INFINITY;
    int i = 0x7fffffff;
    for (int t = threadIdx.x; t < nparts; t += kArgThreads) argmax_merge(v, i, pv[t], pi[t]);
    block_argmax(v, i);
    if (threadIdx.x == 0) {
        if (i == 0x7fffffff) i = 0;  // all NaN: std::max_element returns the first
        *out = i;
        if (tokens && step) {
            tokens[*step] = i;
            *step += 1;
        }
        if (pos) *pos += 1;
    }
}

// ---------------------------------------------------------------------------
// Elementwise
// ---------------------------------------------------------------------------
__global__ void k_add(float* __restrict__ y, const float* __restrict__ a,
                      const float* __restrict__ b, int n) {
    for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < n; t += gridDim.x * blockDim.x)
        y[t] = a[t] + b[t];
}

// silu(x) = x/(1+exp(-x)) (llama_model.cpp:313-315) and elementwise product.
__global__ void k_silu(float* __restrict__ y, const float* __restrict__ x, int n) {
    for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < n; t += gridDim.x * blockDim.x)
        y[t] = x[t] / (1.f + expf(-x[t]));
}

__global__ void k_mul(float* __restrict__ y, const float* __restrict__ a,
                      const float* __restrict__ b, int n) {
    for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < n; t += gridDim.x * blockDim.x)
        y[t] = a[t] * b[t];
}

__global__ void k_set_int(int* p, int v) { *p = v; }

// tokens[*step] = *tok; ++*step  (records the token chosen from the prefill logits)
__global__ void k_push_token(int* tokens, int* step, const int* tok) {
    tokens[*step] = *tok;
    *step += 1;
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
static inline unsigned grid_for(long work, int threads, long cap = 65536) {
    long g = (work + threads - 1) / threads;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (unsigned)g;
}

hipError_t launch_dequant_q4k(float* y, const void* W, long nblocks, hipStream_t st) {
    hipLaunchKernelGGL(k_dequant_q4k, dim3(grid_for(nblocks * 32, 256)), dim3(256), 0, st, y,
                       static_cast<const uint8_t*>(W), nblocks);
    return hipGetLastError();
}
hipError_t launch_dequant_q6k(float* y, const void* W, long nblocks, hipStream_t st) {
    hipLaunchKernelGGL(k_dequant_q6k, dim3(grid_for(nblocks * 16, 256)), dim3(256), 0, st, y,
                       static_cast<const uint8_t*>(W), nblocks);
    return hipGetLastError();
}
hipError_t launch_quantize_q8_0(void* y, const float* x, int n, hipStream_t st) {
    hipLaunchKernelGGL(k_quantize_q8_0, dim3(grid_for(n / 4, 256)), dim3(256), 0, st,
                       static_cast<uint8_t*>(y), x, n);
    return hipGetLastError();
}
hipError_t launch_rmsnorm(float* y, void* yq8, const float* x, const float* w, int n, float eps,
                          hipStream_t st) {
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(kNormThreads), 0, st, y,
                       static_cast<uint8_t*>(yq8), x, w, n, eps);
    return hipGetLastError();
}
hipError_t launch_rmsnorm_rows(float* y, void* yq8, const float* x, const float* w, int n,
                               float eps, int rows, hipStream_t st) {
    hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)rows), dim3(kNormThreads), 0, st, y,
                       static_cast<uint8_t*>(yq8), x, w, n, eps);
    return hipGetLastError();
}
hipError_t launch_rmsnorm_rows_prep(float* y, void* yq8, const float* x, const float* w, int n,
                                    float eps, int T, int Tp, uint8_t* xh, float* dx2, float* gx2,
                                    float* dx4, hipStream_t st) {
    if (n % 32 || n > 32 * kNormThreads || Tp % 64 || T > Tp || T <= 0) return hipErrorInvalidValue;
    // 256 threads (up to 8 float4 each) where the row fits: a quarter of the
    // waves per row (512 rows of 4096: 8.8 -> 8.6 us)
    if (n <= 32 * 256)
        hipLaunchKernelGGL(k_rmsnorm_prep<256>, dim3((unsigned)Tp), dim3(256), 0, st, y,
                           static_cast<uint8_t*>(yq8), x, w, n, eps, T, Tp, xh, dx2, gx2, dx4);
    else
        hipLaunchKernelGGL(k_rmsnorm_prep<kNormThreads>, dim3((unsigned)Tp), dim3(kNormThreads), 0,
                           st, y, static_cast<uint8_t*>(yq8), x, w, n, eps, T, Tp, xh, dx2, gx2,
                           dx4);
    return hipGetLastError();
}
hipError_t launch_rope_kv_rows(const float* k, int k_ld, const float* v, int v_ld,
                               const float* bk, const float* bv, float* kcache, float* vcache,
                               int pos0, int T, int n_kv_heads, int hd, const float* cos_t,
                               const float* sin_t, hipStream_t st) {
    const long work = (long)n_kv_heads * hd / 2 + (long)n_kv_heads * hd;
    const bool vec = hd % 8 == 0 && k_ld % 4 == 0 && v_ld % 4 == 0 &&
                     (((uintptr_t)k | (uintptr_t)v | (uintptr_t)bk | (uintptr_t)bv |
                       (uintptr_t)kcache | (uintptr_t)vcache | (uintptr_t)cos_t |
                       (uintptr_t)sin_t) & 15) == 0;
    if (vec)
        hipLaunchKernelGGL(k_rope_kv_rows4, dim3(grid_for(work / 4, 256, 64), (unsigned)T),
                           dim3(256), 0, st, k, k_ld, v, v_ld, bk, bv, kcache, vcache, pos0,
                           n_kv_heads, hd, cos_t, sin_t);
    else
        hipLaunchKernelGGL(k_rope_kv_rows, dim3(grid_for(work, 256, 64), (unsigned)T), dim3(256),
                           0, st, k, k_ld, v, v_ld, bk, bv, kcache, vcache, pos0, n_kv_heads, hd,
                           cos_t, sin_t);
    return hipGetLastError();
}
hipError_t launch_swiglu_gu(void* outq8, const float* gu, int T, int n, int B, hipStream_t st,
                            float* out) {
    if (n % 32 || B % 4 || n % B) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_swiglu_gu, dim3(grid_for((long)T * n / 4, 256)), dim3(256), 0, st,
                       static_cast<uint8_t*>(outq8), out, gu, T, n, B);
    return hipGetLastError();
}
hipError_t launch_embed_rows(int qtype, float* out, const void* W, const int* toks_dev, int T,
                             int nb, long row_bytes, hipStream_t st) {
    if (qtype == 12)
        hipLaunchKernelGGL(k_embed_q4k, dim3((unsigned)T), dim3(1024), 0, st, out,
                           static_cast<const uint8_t*>(W), toks_dev, 0, nb, row_bytes);
    else
        hipLaunchKernelGGL(k_embed_q6k, dim3((unsigned)T), dim3(1024), 0, st, out,
                           static_cast<const uint8_t*>(W), toks_dev, 0, nb, row_bytes);
    return hipGetLastError();
}
hipError_t launch_rope(float* dst, const float* src, const int* pos_dev, int pos, int n_heads,
                       int hd, const float* cos_t, const float* sin_t, hipStream_t st) {
    hipLaunchKernelGGL(k_rope, dim3(grid_for((long)n_heads * hd / 2, 256, 1024)), dim3(256), 0,
                       st, dst, src, pos_dev, pos, n_heads, hd, cos_t, sin_t);
    return hipGetLastError();
}
hipError_t launch_rope_qkv(float* q, const float* k, const float* v, float* kcache,
                           float* vcache, const int* pos_dev, int pos, int n_heads,
                           int n_kv_heads, int hd, const float* cos_t, const float* sin_t,
                           hipStream_t st) {
    const long work = (long)(n_heads + n_kv_heads) * hd / 2 + (long)n_kv_heads * hd;
    hipLaunchKernelGGL(k_rope_qkv, dim3(grid_for(work, 256, 1024)), dim3(256), 0, st, q, k, v,
                       kcache, vcache, pos_dev, pos, n_heads, n_kv_heads, hd, cos_t, sin_t);
    return hipGetLastError();
}

hipError_t launch_swiglu(float* out, void* outq8, const float* gate, const float* up, int n,
                         hipStream_t st) {
    hipLaunchKernelGGL(k_swiglu, dim3(grid_for(n / 4, 256)), dim3(256), 0, st, out,
                       static_cast<uint8_t*>(outq8), gate, up, n);
    return hipGetLastError();
}

hipError_t launch_embed(int qtype, float* out, const void* W, const int* tok_dev, int tok,
                        int nb, long row_bytes, hipStream_t st) {
    if (qtype == 12)
        hipLaunchKernelGGL(k_embed_q4k, dim3(1), dim3(1024), 0, st, out,
                           static_cast<const uint8_t*>(W), tok_dev, tok, nb, row_bytes);
    else
        hipLaunchKernelGGL(k_embed_q6k, dim3(1), dim3(1024), 0, st, out,
                           static_cast<const uint8_t*>(W), tok_dev, tok, nb, row_bytes);
    return hipGetLastError();
}

constexpr int kArgParts = 256;
int argmax_parts() { return kArgParts; }

hipError_t launch_argmax_final(int* out, const float* pv, const int* pi, int nparts, int* tokens,
                               int* step, int* pos, hipStream_t st) {
    if (nparts <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(kArgThreads), 0, st, out, pv, pi, nparts,
                       tokens, step, pos);
    return hipGetLastError();
}

hipError_t launch_argmax(int* out, float* pv, int* pi, const float* x, int n, int* tokens,
                         int* step, int* pos, hipStream_t st) {
    const int parts = (int)grid_for(n, kArgThreads, kArgParts);
    hipLaunchKernelGGL(k_argmax_partial, dim3(parts), dim3(kArgThreads), 0, st, pv, pi, x, n);
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(kArgThreads), 0, st, out, pv, pi, parts,
                       tokens, step, pos);
    return hipGetLastError();
}

hipError_t launch_add(float* y, const float* a, const float* b, int n, hipStream_t st) {
    hipLaunchKernelGGL(k_add, dim3(grid_for(n, 256)), dim3(256), 0, st, y, a, b, n);
    return hipGetLastError();
}

hipError_t launch_silu(float* y, const float* x, int n, hipStream_t st) {
    hipLaunchKernelGGL(k_silu, dim3(grid_for(n, 256)), dim3(256), 0, st, y, x, n);
    return hipGetLastError();
}

hipError_t launch_mul(float* y, const float* a, const float* b, int n, hipStream_t st) {
    hipLaunchKernelGGL(k_mul, dim3(grid_for(n, 256)), dim3(256), 0, st, y, a, b, n);
    return hipGetLastError();
}

hipError_t launch_set_int(int* p, int v, hipStream_t st) {
    hipLaunchKernelGGL(k_set_int, dim3(1), dim3(1), 0, st, p, v);
    return hipGetLastError();
}

hipError_t launch_push_token(int* tokens, int* step, const int* tok, hipStream_t st) {
    hipLaunchKernelGGL(k_push_token, dim3(1), dim3(1), 0, st, tokens, step, tok);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Plain streaming read (a measurement kernel): every 16-byte vector of
// [p, p + n16*16) is loaded once; thread i of a grid of G threads loads
// vectors i, i + G, ... (U of them in flight per loop trip: one wave
// instruction covers 1 KiB of contiguous bytes) and XORs them.  Nothing is
// written unless the XOR equals a magic value, so the kernel's bytes are the
// reads alone: the practical read ceiling of a launch of this size.
// ---------------------------------------------------------------------------
template <int U>
__global__ __launch_bounds__(256) void k_stream_read(const uint4* __restrict__ p, long n16,
                                                     uint32_t* __restrict__ sink) {
    const long G = (long)gridDim.x * 256;
    uint32_t acc = 0;
    for (long i0 = (long)blockIdx.x * 256 + threadIdx.x; i0 < n16; i0 += G * U) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = p[min(i0 + u * G, n16 - 1)];
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

hipError_t launch_stream_read(const void* p, size_t bytes, int unroll, int wgs, uint32_t* sink,
                              hipStream_t st) {
    const long n16 = (long)(bytes / 16);
    if (n16 <= 0 || wgs <= 0) return hipErrorInvalidValue;
    const auto* q = static_cast<const uint4*>(p);
    switch (unroll) {
        case 1: hipLaunchKernelGGL(k_stream_read<1>, dim3(wgs), dim3(256), 0, st, q, n16, sink); break;
        case 2: hipLaunchKernelGGL(k_stream_read<2>, dim3(wgs), dim3(256), 0, st, q, n16, sink); break;
        case 4: hipLaunchKernelGGL(k_stream_read<4>, dim3(wgs), dim3(256), 0, st, q, n16, sink); break;
        case 8: hipLaunchKernelGGL(k_stream_read<8>, dim3(wgs), dim3(256), 0, st, q, n16, sink); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace axf
