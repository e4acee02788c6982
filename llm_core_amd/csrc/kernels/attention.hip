// attention.hip — single-token GQA attention over the fp32 KV cache, fused
// with RoPE of the new query and RoPE + store of the new key/value row
// (llama_forward_token, llama_model.cpp:1241-1272).
//
// Two kernels:
//   k_attn_split   grid (nsplit, n_kv_heads).  Workgroup (j, kvh) serves the
//                  G = n_heads / n_kv_heads query heads of kv head kvh over
//                  positions [j*S, min(j*S+S, seq)), S = kAttnSplit, so every
//                  K/V row is read once per group.  All K and V loads of the
//                  tile are issued before any arithmetic (the tile lives in
//                  registers), so a workgroup pays one HBM round trip.  It
//                  writes, per head, the split's max score m_j, the sum
//                  l_j = sum exp(s - m_j) and o_j = sum exp(s - m_j) v.
//                  Splits past the current position exit at once, so the grid
//                  can be sized for the whole context and replayed.
//   k_attn_combine grid (n_heads).  out = sum_j o_j e^(m_j - M) / sum_j l_j e^(m_j - M),
//                  M = max_j m_j, over the non-empty splits, plus the Q8_0
//                  blocks of out for the next projection.
// s = dot(q_h, k_t) / sqrt(HD).  The split containing the current position
// also RoPEs the new key (+ bias), stores it and the new value (+ bias) to the
// caches, and uses them for that row.
//
// The kernel boundary between the two orders the partials: on gfx950 each
// XCD has its own L2, and an in-kernel device-scope fence costs an L2
// writeback + invalidate per workgroup.
#include "common.hpp"

namespace axf {

constexpr int kAttnSplit = 64;  // positions per workgroup (= one wave's lanes)
constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr int kMaxSplit = 512;  // contexts up to 32768 positions

template <int HD>
__device__ __forceinline__ void rope_in_lds(float* v, int n_vec, const float* cr, const float* sr) {
    constexpr int half = HD / 2;
    for (int t = threadIdx.x; t < n_vec * half; t += kAttnThreads) {
        const int g = t / half, i = t % half;
        float* h = v + g * HD;
        const float x0 = h[i], x1 = h[i + half];
        const float c = cr[i], s = sr[i];
        h[i] = fmaf(x0, c, -(x1 * s));
        h[i + half] = fmaf(x0, s, x1 * c);
    }
}

// Q8_0 of 32 values held as float4 by 8 consecutive lanes (sub = lane & 7).
__device__ __forceinline__ void q8_store4(uint8_t* blk, int sub, float4 v) {
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
    const float d = amax / 127.f;
    const float id = amax > 0.f ? 127.f / amax : 0.f;
    auto q = [&](float f) -> uint32_t {
        float r = rintf(f * id);
        r = fminf(fmaxf(r, -128.f), 127.f);
        return (uint32_t)((int)r & 0xff);
    };
    *reinterpret_cast<uint32_t*>(blk + 4 + 4 * sub) =
        q(v.x) | (q(v.y) << 8) | (q(v.z) << 16) | (q(v.w) << 24);
    if (sub == 0) *reinterpret_cast<float*>(blk) = d;
}

__device__ __forceinline__ float dot4f(float4 a, float4 b, float acc) {
    acc = fmaf(a.x, b.x, acc);
    acc = fmaf(a.y, b.y, acc);
    acc = fmaf(a.z, b.z, acc);
    return fmaf(a.w, b.w, acc);
}

__device__ __forceinline__ float4 fma4(float s, float4 v, float4 o) {
    return make_float4(fmaf(s, v.x, o.x), fmaf(s, v.y, o.y), fmaf(s, v.z, o.z), fmaf(s, v.w, o.w));
}

// G = query heads per kv head (compile-time upper bound GM, runtime g < G).
// Lane layout of the K/V tile: a row of HD floats is read by LPR = HD/4 lanes
// (one float4 each); one wave instruction covers RPI = 64/LPR rows; wave w owns
// rows [w*RPW, w*RPW + RPW) of the split.
template <int HD, int GM>
__global__ __launch_bounds__(kAttnThreads) void k_attn_split(AttnArgs a) {
    constexpr int LPR = HD / 4;
    constexpr int RPI = 64 / LPR;
    constexpr int RPW = kAttnSplit / kAttnWaves;
    constexpr int NI = RPW / RPI;
    static_assert(RPW % RPI == 0, "tile shape");
    __shared__ float qs[GM * HD];
    __shared__ float knew[HD], vnew[HD];
    __shared__ float sc[GM][kAttnSplit];
    __shared__ float ov[kAttnWaves][GM * HD];
    __shared__ float stat[GM][2];

    const int j = blockIdx.x, kvh = blockIdx.y;
    const int G = a.n_heads / a.n_kv_heads;
    const int p = a.pos_dev ? *a.pos_dev : a.pos;
    const int t0 = j * kAttnSplit;
    if (t0 > p) return;  // split past the current position: nothing to do
    const int n = min(kAttnSplit, p + 1 - t0);
    const size_t kve = (size_t)a.n_kv_heads * HD;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = (lane % LPR) * 4, rsub = lane / LPR;
    const bool owns_new = a.store_kv && p - t0 < kAttnSplit;

    // 1. the whole K/V tile into registers (rows past n and the new row read as 0)
    float4 kr[NI], vr[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int r = wave * RPW + i * RPI + rsub;
        const int t = t0 + r;
        kr[i] = vr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < n && !(owns_new && t == p)) {
            const size_t off = (size_t)t * kve + (size_t)kvh * HD + col;
            kr[i] = *reinterpret_cast<const float4*>(a.kcache + off);
            vr[i] = *reinterpret_cast<const float4*>(a.vcache + off);
        }
    }

    // 2. query heads of this group (+ bias), new key/value (+ bias), RoPE
    for (int t = threadIdx.x; t < G * HD; t += kAttnThreads) {
        const size_t h = (size_t)kvh * G + t / HD;
        const int d = t % HD;
        float v = a.q[h * HD + d];
        if (a.bq) v += a.bq[h * HD + d];
        qs[t] = v;
    }
    if (owns_new) {
        for (int d = threadIdx.x; d < HD; d += kAttnThreads) {
            float kk = a.k[(size_t)kvh * HD + d], vv = a.v[(size_t)kvh * HD + d];
            if (a.bk) kk += a.bk[(size_t)kvh * HD + d];
            if (a.bv) vv += a.bv[(size_t)kvh * HD + d];
            knew[d] = kk;
            vnew[d] = vv;
        }
    }
    __syncthreads();
    if (a.cos_t) {
        const float* cr = a.cos_t + (size_t)p * (HD / 2);
        const float* sr = a.sin_t + (size_t)p * (HD / 2);
        rope_in_lds<HD>(qs, G, cr, sr);
        if (owns_new) rope_in_lds<HD>(knew, 1, cr, sr);
    }
    __syncthreads();
    if (owns_new) {
        for (int d = threadIdx.x; d < HD; d += kAttnThreads) {
            a.kcache[(size_t)p * kve + (size_t)kvh * HD + d] = knew[d];
            a.vcache[(size_t)p * kve + (size_t)kvh * HD + d] = vnew[d];
        }
#pragma unroll
        for (int i = 0; i < NI; i++) {
            if (t0 + wave * RPW + i * RPI + rsub == p) {
                kr[i] = *reinterpret_cast<const float4*>(knew + col);
                vr[i] = *reinterpret_cast<const float4*>(vnew + col);
            }
        }
    }

    // 3. scores
    const float scale = 1.f / sqrtf((float)HD);
    float4 qv[GM];
#pragma unroll
    for (int g = 0; g < GM; g++)
        qv[g] = g < G ? *reinterpret_cast<const float4*>(qs + g * HD + col)
                      : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int r = wave * RPW + i * RPI + rsub;
#pragma unroll
        for (int g = 0; g < GM; g++) {
            if (g < G) {
                const float s = group_sum<LPR>(dot4f(qv[g], kr[i], 0.f));
                if (lane % LPR == 0) sc[g][r] = r < n ? s * scale : -INFINITY;
            }
        }
    }
    __syncthreads();

    // 4. per-head max, exp, sum: wave w takes heads w, w+4, ...; lane = row
    for (int g = wave; g < G; g += kAttnWaves) {
        const float s = sc[g][lane];
        const float m = wave_max(s);
        const float e = lane < n ? expf(s - m) : 0.f;
        sc[g][lane] = e;
        const float l = wave_sum(e);
        if (lane == 0) {
            stat[g][0] = m;
            stat[g][1] = l;
        }
    }
    __syncthreads();

    // 5. values: lane-local rows, then across the RPI rows of an instruction, then waves
    float4 o[GM];
#pragma unroll
    for (int g = 0; g < GM; g++) o[g] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int r = wave * RPW + i * RPI + rsub;
#pragma unroll
        for (int g = 0; g < GM; g++)
            if (g < G) o[g] = fma4(sc[g][r], vr[i], o[g]);
    }
#pragma unroll
    for (int g = 0; g < GM; g++) {
        if (g < G) {
#pragma unroll
            for (int off = LPR; off < 64; off <<= 1) {
                o[g].x += __shfl_xor(o[g].x, off);
                o[g].y += __shfl_xor(o[g].y, off);
                o[g].z += __shfl_xor(o[g].z, off);
                o[g].w += __shfl_xor(o[g].w, off);
            }
            if (rsub == 0) *reinterpret_cast<float4*>(&ov[wave][g * HD + col]) = o[g];
        }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < G * HD; t += kAttnThreads) {
        const int g = t / HD, d = t % HD;
        float acc = ov[0][t];
#pragma unroll
        for (int w = 1; w < kAttnWaves; w++) acc += ov[w][t];
        a.part[((size_t)(kvh * G + g) * a.nsplit + j) * (HD + 2) + 2 + d] = acc;
    }
    if (threadIdx.x < G) {
        float* dst = a.part + ((size_t)(kvh * G + threadIdx.x) * a.nsplit + j) * (HD + 2);
        dst[0] = stat[threadIdx.x][0];
        dst[1] = stat[threadIdx.x][1];
    }
}

// One workgroup per query head.  Thread t accumulates float4 column t % (HD/4)
// over the splits js, js + NJS, ... (js = t / (HD/4)); the NJS partial sums are
// added in LDS.
template <int HD>
__global__ __launch_bounds__(kAttnThreads) void k_attn_combine(AttnArgs a) {
    constexpr int C4 = HD / 4;
    constexpr int NJS = kAttnThreads / C4;
    __shared__ float wsplit[kMaxSplit];
    __shared__ float red[kAttnWaves];
    __shared__ float4 acc4[NJS][C4];
    __shared__ float outv[HD];

    const int h = blockIdx.x;
    const int p = a.pos_dev ? *a.pos_dev : a.pos;
    const int ns = p / kAttnSplit + 1;  // non-empty splits
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float* ph = a.part + (size_t)h * a.nsplit * (HD + 2);

    float mx = -INFINITY;
    for (int jj = threadIdx.x; jj < ns; jj += kAttnThreads) mx = fmaxf(mx, ph[(size_t)jj * (HD + 2)]);
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < kAttnWaves; w++) M = fmaxf(M, red[w]);
    __syncthreads();
    float lsum = 0.f;
    for (int jj = threadIdx.x; jj < ns; jj += kAttnThreads) {
        const float w = expf(ph[(size_t)jj * (HD + 2)] - M);
        wsplit[jj] = w;
        lsum = fmaf(ph[(size_t)jj * (HD + 2) + 1], w, lsum);
    }
    lsum = wave_sum(lsum);
    if (lane == 0) red[wave] = lsum;
    __syncthreads();
    float L = red[0];
#pragma unroll
    for (int w = 1; w < kAttnWaves; w++) L += red[w];

    const int c = threadIdx.x % C4, js = threadIdx.x / C4;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    int jj = js;
    for (; jj + 3 * NJS < ns; jj += 4 * NJS) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++)
            v[u] = *reinterpret_cast<const float4*>(ph + (size_t)(jj + u * NJS) * (HD + 2) + 2 + 4 * c);
#pragma unroll
        for (int u = 0; u < 4; u++) acc = fma4(wsplit[jj + u * NJS], v[u], acc);
    }
    for (; jj < ns; jj += NJS)
        acc = fma4(wsplit[jj], *reinterpret_cast<const float4*>(ph + (size_t)jj * (HD + 2) + 2 + 4 * c), acc);
    acc4[js][c] = acc;
    __syncthreads();
    const float invL = 1.f / L;
    for (int d = threadIdx.x; d < HD; d += kAttnThreads) {
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < NJS; q++) s += reinterpret_cast<const float*>(&acc4[q][0])[d];
        const float r = s * invL;
        a.out[(size_t)h * HD + d] = r;
        outv[d] = r;
    }
    if (a.outq8) {
        __syncthreads();
        if (threadIdx.x < C4) {
            const float4 v = *reinterpret_cast<const float4*>(outv + 4 * threadIdx.x);
            const size_t e0 = (size_t)h * HD + 4 * threadIdx.x;
            q8_store4(a.outq8 + (e0 >> 5) * Q8_0_BYTES, threadIdx.x & 7, v);
        }
    }
}

int attn_nsplit(int max_seq) { return (max_seq + kAttnSplit - 1) / kAttnSplit; }

template <int HD>
static hipError_t launch_attn_hd(const AttnArgs& a, int G, hipStream_t st) {
    const dim3 grid((unsigned)a.nsplit, (unsigned)a.n_kv_heads);
    if (G == 1)
        hipLaunchKernelGGL((k_attn_split<HD, 1>), grid, dim3(kAttnThreads), 0, st, a);
    else if (G == 2)
        hipLaunchKernelGGL((k_attn_split<HD, 2>), grid, dim3(kAttnThreads), 0, st, a);
    else if (G <= 4)
        hipLaunchKernelGGL((k_attn_split<HD, 4>), grid, dim3(kAttnThreads), 0, st, a);
    else if (G <= 8)
        hipLaunchKernelGGL((k_attn_split<HD, 8>), grid, dim3(kAttnThreads), 0, st, a);
    else
        return hipErrorInvalidValue;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_attn_combine<HD>), dim3((unsigned)a.n_heads), dim3(kAttnThreads), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_attention_fused(const AttnArgs& a, int head_dim, hipStream_t st) {
    if (a.n_kv_heads <= 0 || a.n_heads % a.n_kv_heads) return hipErrorInvalidValue;
    const int G = a.n_heads / a.n_kv_heads;
    if (a.nsplit < 1 || a.nsplit > kMaxSplit || G > 8 || (a.store_kv && !a.cos_t))
        return hipErrorInvalidValue;
    switch (head_dim) {
        case 64: return launch_attn_hd<64>(a, G, st);
        case 128: return launch_attn_hd<128>(a, G, st);
        case 256: return launch_attn_hd<256>(a, G, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace axf
