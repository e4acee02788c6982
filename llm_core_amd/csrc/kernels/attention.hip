// attention.hip — single-token GQA attention over the fp32 KV cache, fused
// with RoPE of the new query and RoPE + store of the new key/value row
// (llama_forward_token, llama_model.cpp:1241-1272).
//
// Two kernels:
//   k_attn_split   grid (n_kv_heads, nsplit).  Workgroup (kvh, j) serves the
//                  G = n_heads / n_kv_heads query heads of kv head kvh over
//                  positions [j*S, min(j*S+S, seq)), S = kAttnSplit, so every
//                  K/V row is read once per group.  All K and V loads of the
//                  tile are issued right after the small operands (query,
//                  new K/V row, RoPE row) and before any arithmetic (the tile
//                  lives in registers), so a workgroup pays one HBM round trip.  It
//                  writes, per head, the split's max score m_j, the sum
//                  l_j = sum exp(s - m_j) and o_j = sum exp(s - m_j) v.
//                  Splits past the current position exit at once, so the grid
//                  can be sized for the whole context and replayed.
//   k_attn_combine grid (n_heads).  out = sum_j o_j e^(m_j - M) / sum_j l_j e^(m_j - M),
//                  M = max_j m_j (found first), over the non-empty splits,
//                  plus the Q8_0 blocks of out for the next projection.
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

// rotate-half RoPE of n_vec head vectors held in LDS; cr/sr: this position's
// table row (LDS)
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

// Per-head q/k RMSNorm (qwen3: before RoPE, hunyuan-dense: after it) with
// the bias, RoPE and the K/V store: workgroup (head hh, row t) of 64 threads
// finishes query head hh (hh < H, in place) or kv head hh - H (K and V rows
// into the caches at position pos + t).  The attention kernels then run
// with no bias, no RoPE and no store.  The norm is rms_norm_avx2's
// (llama_model.cpp:371-393): 8 partial sums, partial j the fma chain over
// elements j, j+8, ... in order, added 0 + p0 + ... + p7, then
// 1/sqrt(ss/n + eps), x = w * (x * scale); RoPE as rope_in_lds.
__global__ __launch_bounds__(64) void k_qk_prep(QkPrepArgs a) {
    __shared__ float buf[256];
    __shared__ float part[9];
    const int hh = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, HD = a.hd, half = HD / 2;
    const int pos = (a.pos_dev ? *a.pos_dev : a.pos) + t;
    const bool isq = hh < a.n_heads;
    const int kh = hh - a.n_heads;
    const size_t kve = (size_t)a.n_kv_heads * HD;
    const float* src = isq ? a.q + (size_t)t * a.q_ld + (size_t)hh * HD
                           : a.k + (size_t)t * a.k_ld + (size_t)kh * HD;
    const float* bias = isq ? (a.bq ? a.bq + (size_t)hh * HD : nullptr)
                            : (a.bk ? a.bk + (size_t)kh * HD : nullptr);
    const float* w = isq ? a.qn : a.kn;
    float* dst = isq ? a.q + (size_t)t * a.q_ld + (size_t)hh * HD
                     : a.kcache + (size_t)pos * kve + (size_t)kh * HD;
    for (int i = tid; i < HD; i += 64) buf[i] = bias ? src[i] + bias[i] : src[i];
    if (!isq) {  // V row (+ bias), unrotated and not normalised
        const float* vs = a.v + (size_t)t * a.v_ld + (size_t)kh * HD;
        float* vd = a.vcache + (size_t)pos * kve + (size_t)kh * HD;
        for (int i = tid; i < HD; i += 64) vd[i] = a.bv ? vs[i] + a.bv[(size_t)kh * HD + i] : vs[i];
    }
    __syncthreads();
    auto norm = [&]() {
        if (!w) return;
        if (tid < 8) {
            float acc = 0.f;
            for (int i = tid; i < HD; i += 8) acc = fmaf(buf[i], buf[i], acc);
            part[tid] = acc;
        }
        __syncthreads();
        if (tid == 0) {
            float ss = 0.f;
            for (int j = 0; j < 8; j++) ss += part[j];
            part[8] = 1.f / sqrtf(ss / (float)HD + a.eps);
        }
        __syncthreads();
        const float r = part[8];
        for (int i = tid; i < HD; i += 64) buf[i] = w[i] * (buf[i] * r);
        __syncthreads();
    };
    auto rope = [&]() {
        const float* cr = a.cos_t + (size_t)pos * half;
        const float* sr = a.sin_t + (size_t)pos * half;
        for (int i = tid; i < half; i += 64) {
            const float x0 = buf[i], x1 = buf[i + half], c = cr[i], sn = sr[i];
            buf[i] = fmaf(x0, c, -(x1 * sn));
            buf[i + half] = fmaf(x0, sn, x1 * c);
        }
        __syncthreads();
    };
    if (a.order == 1) norm();
    rope();
    if (a.order == 2) norm();
    for (int i = tid; i < HD; i += 64) dst[i] = buf[i];
}

// Q8_0 of 32 values held as float4 by 8 consecutive lanes (sub = lane & 7).
__device__ __forceinline__ void q8_store4(uint8_t* blk, int sub, float4 v) {
    float d;
    *reinterpret_cast<uint32_t*>(blk + 4 + 4 * sub) = q8_quant4(v, d);
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
    constexpr int QPT = (GM * HD + kAttnThreads - 1) / kAttnThreads;
    static_assert(HD <= kAttnThreads, "one new K/V element per thread");
    __shared__ float qs[GM * HD];
    __shared__ float knew[HD], vnew[HD];
    __shared__ float crs[HD / 2], srs[HD / 2];
    __shared__ float sc[GM][kAttnSplit];
    __shared__ float ov[kAttnWaves][GM * HD];
    __shared__ float stat[GM][2];

    // kv head fastest: workgroups dispatched together read adjacent bytes of each
    // KV row.  blockIdx.x = kv head * groups + group: a workgroup serves query
    // heads g0 .. g0+Gl-1 of its kv head (GM per group; several groups re-read
    // the same K/V rows, from L2, when there are few kv heads and splits).
    const int G = a.n_heads / a.n_kv_heads;
    const int ngrp = (G + GM - 1) / GM;
    const int kvh = blockIdx.x / ngrp, g0 = (blockIdx.x % ngrp) * GM;
    const int Gl = min(GM, G - g0);
    const int j = blockIdx.y, tok = blockIdx.z;
    const int p = (a.pos_dev ? *a.pos_dev : a.pos) + tok;
    // query row tok and its partials (tok > 0 only in batched prefill)
    const float* qp = a.q + (size_t)tok * a.q_ld;
    float* part = a.part + (size_t)tok * a.n_heads * a.nsplit * (HD + 2);
    const int t0 = j * kAttnSplit;
    if (t0 > p) return;  // split past the current position: nothing to do
    const int n = min(kAttnSplit, p + 1 - t0);
    const size_t kve = (size_t)a.n_kv_heads * HD;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = (lane % LPR) * 4, rsub = lane / LPR;
    // the split holding the new row uses it; the first head group stores it
    const bool owns_new = a.store_kv && p - t0 < kAttnSplit;
    const bool stores_new = owns_new && g0 == 0;
    const int tid = threadIdx.x;

    // 1. small operands first, so their latency hides under the tile loads:
    //    query (and bias) elements, the new key/value row, this position's RoPE
    //    row.  Every load below is unconditional (clamped, in-bounds addresses;
    //    unused values are discarded by selects), so the compiler can wait for
    //    exactly the loads each use needs instead of draining the tile.
    float qraw[QPT], qb[QPT];
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int t = min(tid + k * kAttnThreads, Gl * HD - 1);
        const size_t e = ((size_t)kvh * G + g0 + t / HD) * HD + t % HD;
        qraw[k] = qp[e];
        qb[k] = (a.bq ? a.bq : qp)[e];
    }
    const int d1 = min(tid, HD - 1);
    const size_t e1 = (size_t)kvh * HD + d1;  // < n_kv_heads * HD <= n_heads * HD
    const float kk = (a.store_kv ? a.k : qp)[e1];
    const float vv = (a.store_kv ? a.v : qp)[e1];
    const float kb = (a.bk ? a.bk : qp)[e1];
    const float vb = (a.bv ? a.bv : qp)[e1];
    const int d2 = min(tid, HD / 2 - 1);
    const float cv = a.cos_t ? a.cos_t[(size_t)p * (HD / 2) + d2] : 0.f;
    const float sv = a.cos_t ? a.sin_t[(size_t)p * (HD / 2) + d2] : 0.f;

    // 2. the whole K/V tile into registers.  Rows past n re-read row t0 (a
    //    written, finite row); their score is -inf and their weight 0 below.
    //    The new row p (still stale in the cache) is replaced after the RoPE.
    //    K rows first: the scores and the softmax need only them, and run
    //    while the V rows are still arriving.
    float4 kr[NI], vr[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int r = wave * RPW + i * RPI + rsub;
        const size_t off = (size_t)(r < n ? t0 + r : t0) * kve + (size_t)kvh * HD + col;
        kr[i] = *reinterpret_cast<const float4*>(a.kcache + off);
    }
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int r = wave * RPW + i * RPI + rsub;
        const size_t off = (size_t)(r < n ? t0 + r : t0) * kve + (size_t)kvh * HD + col;
        vr[i] = *reinterpret_cast<const float4*>(a.vcache + off);
    }

    // 3. bias and RoPE in LDS, store the new K/V row
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int t = tid + k * kAttnThreads;
        if (t < Gl * HD) qs[t] = a.bq ? qraw[k] + qb[k] : qraw[k];
    }
    if (owns_new && tid < HD) {
        knew[tid] = a.bk ? kk + kb : kk;
        vnew[tid] = a.bv ? vv + vb : vv;
    }
    if (a.cos_t && tid < HD / 2) {
        crs[tid] = cv;
        srs[tid] = sv;
    }
    __syncthreads();
    if (a.cos_t) {
        rope_in_lds<HD>(qs, Gl, crs, srs);
        if (owns_new) rope_in_lds<HD>(knew, 1, crs, srs);
    }
    __syncthreads();
    if (owns_new) {
        if (stores_new && tid < HD) {
            a.kcache[(size_t)p * kve + (size_t)kvh * HD + tid] = knew[tid];
            a.vcache[(size_t)p * kve + (size_t)kvh * HD + tid] = vnew[tid];
        }
#pragma unroll
        for (int i = 0; i < NI; i++) {
            if (t0 + wave * RPW + i * RPI + rsub == p) {
                kr[i] = *reinterpret_cast<const float4*>(knew + col);
                vr[i] = *reinterpret_cast<const float4*>(vnew + col);
            }
        }
    }

    // 4. scores
    const float scale = 1.f / sqrtf((float)HD);
    float4 qv[GM];
#pragma unroll
    for (int g = 0; g < GM; g++)
        qv[g] = g < Gl ? *reinterpret_cast<const float4*>(qs + g * HD + col)
                      : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int r = wave * RPW + i * RPI + rsub;
#pragma unroll
        for (int g = 0; g < GM; g++) {
            if (g < Gl) {
                // DPP reduction: the row's sum lands in its last lane
                const float s = group_sum_last<LPR>(dot4f(qv[g], kr[i], 0.f));
                if (lane % LPR == LPR - 1) sc[g][r] = r < n ? s * scale : -INFINITY;
            }
        }
    }
    __syncthreads();

    // 5. per-head max, exp, sum: wave w takes heads w, w+4, ...; lane = row
    for (int g = wave; g < Gl; g += kAttnWaves) {
        const float s = sc[g][lane];
        const float m = wave_max_bcast(s);
        const float e = lane < n ? expf(s - m) : 0.f;
        sc[g][lane] = e;
        const float l = group_sum_last<64>(e);
        if (lane == 63) {
            stat[g][0] = m;
            stat[g][1] = l;
        }
    }
    __syncthreads();

    // 6. values: lane-local rows, then across the RPI rows of an instruction, then waves
    float4 o[GM];
#pragma unroll
    for (int g = 0; g < GM; g++) o[g] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int r = wave * RPW + i * RPI + rsub;
#pragma unroll
        for (int g = 0; g < GM; g++)
            if (g < Gl) o[g] = fma4(sc[g][r], vr[i], o[g]);
    }
#pragma unroll
    for (int g = 0; g < GM; g++) {
        if (g < Gl) {
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
    for (int t = threadIdx.x; t < Gl * HD; t += kAttnThreads) {
        const int g = t / HD, d = t % HD;
        float acc = ov[0][t];
#pragma unroll
        for (int w = 1; w < kAttnWaves; w++) acc += ov[w][t];
        part[((size_t)(kvh * G + g0 + g) * a.nsplit + j) * (HD + 2) + 2 + d] = acc;
    }
    if ((int)threadIdx.x < Gl) {
        float* dst = part + ((size_t)(kvh * G + g0 + threadIdx.x) * a.nsplit + j) * (HD + 2);
        dst[0] = stat[threadIdx.x][0];
        dst[1] = stat[threadIdx.x][1];
    }
}

// One workgroup per query head.  Thread t owns float4 column c = t % (HD/4)
// and the splits js, js + NJS, ... (js = t / (HD/4)).  The loads of its first
// U splits (m, l, o) are issued before anything else.  The workgroup first
// finds M = max_j m_j over the non-empty splits (wave maxima through LDS), so
// every split's weight e^(m_j - M) is independent of the others: each thread
// sums w_j o_j and w_j l_j over its splits, and the NJS partial sums of a
// column are added in a fixed order in LDS:
//   out = sum_j o_j e^(m_j - M) / sum_j l_j e^(m_j - M).
template <int HD>
__global__ __launch_bounds__(kAttnThreads) void k_attn_combine(AttnArgs a) {
    constexpr int C4 = HD / 4;
    constexpr int NJS = kAttnThreads / C4;
    constexpr int U = 4;  // splits loaded per step
    __shared__ float4 accs[NJS][C4];
    __shared__ float ls[NJS];
    __shared__ float wmax[kAttnWaves];

    const int h = blockIdx.x, tok = blockIdx.y;
    const int p = (a.pos_dev ? *a.pos_dev : a.pos) + tok;
    const int ns = p / kAttnSplit + 1;  // non-empty splits
    const float* ph = a.part + ((size_t)tok * a.n_heads + h) * a.nsplit * (HD + 2);
    const int c = threadIdx.x % C4, js = threadIdx.x / C4;

    // this thread's first U splits; splits past ns re-read split ns-1 (written)
    // and are dropped below
    float mj[U], lj[U];
    float4 oj[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const float* pj = ph + (size_t)min(js + u * NJS, ns - 1) * (HD + 2);
        mj[u] = pj[0];
        lj[u] = pj[1];
        oj[u] = make_float4(pj[2 + 4 * c], pj[3 + 4 * c], pj[4 + 4 * c], pj[5 + 4 * c]);
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int u = 0; u < U; u++)
        if (js + u * NJS < ns) mloc = fmaxf(mloc, mj[u]);
    for (int jj = js + U * NJS; jj < ns; jj += NJS) mloc = fmaxf(mloc, ph[(size_t)jj * (HD + 2)]);
    const float wm = wave_max_bcast(mloc);
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = wm;
    __syncthreads();
    float M = wmax[0];
#pragma unroll
    for (int w = 1; w < kAttnWaves; w++) M = fmaxf(M, wmax[w]);

    float l = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < U; u++) {
        if (js + u * NJS < ns) {
            const float w = expf(mj[u] - M);
            l = fmaf(lj[u], w, l);
            acc = fma4(w, oj[u], acc);
        }
    }
    // contexts beyond U * NJS splits
    for (int j0 = js + U * NJS; j0 < ns; j0 += U * NJS) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const float* pj = ph + (size_t)min(j0 + u * NJS, ns - 1) * (HD + 2);
            mj[u] = pj[0];
            lj[u] = pj[1];
            oj[u] = make_float4(pj[2 + 4 * c], pj[3 + 4 * c], pj[4 + 4 * c], pj[5 + 4 * c]);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (j0 + u * NJS < ns) {
                const float w = expf(mj[u] - M);
                l = fmaf(lj[u], w, l);
                acc = fma4(w, oj[u], acc);
            }
        }
    }
    accs[js][c] = acc;
    if (c == 0) ls[js] = l;
    __syncthreads();
    if (threadIdx.x < C4) {
        float L = 0.f;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int q = 0; q < NJS; q++) {
            L += ls[q];
            const float4 aq = accs[q][c];
            o = make_float4(o.x + aq.x, o.y + aq.y, o.z + aq.z, o.w + aq.w);
        }
        const float inv = 1.f / L;
        o = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
        float* dst = a.out + (size_t)tok * a.out_ld + (size_t)h * HD + 4 * c;
        dst[0] = o.x;
        dst[1] = o.y;
        dst[2] = o.z;
        dst[3] = o.w;
        if (a.outq8) {
            // lanes 0..C4-1 of wave 0: 8 consecutive lanes hold one 32-value block
            const size_t e0 = (size_t)tok * a.out_ld + (size_t)h * HD + 4 * c;
            q8_store4(a.outq8 + (e0 >> 5) * Q8_0_BYTES, c & 7, o);
        }
    }
}

// ---------------------------------------------------------------------------
// Batched prefill attention on the matrix cores (llama_forward_batch's causal
// attention, src/models/llama_model.cpp:1410-1426): a workgroup owns 64 query
// rows of one kv head (QT = 64 / G tokens x the G query heads that share it)
// and walks the keys 0 .. (its last token's position) in blocks of 32.  Each
// K/V block is staged once in LDS and used by all 64 rows:
//   S = Q K^T   v_mfma_f32_16x16x4_f32, A = the wave's 16 query rows (held in
//               VGPRs, bias and RoPE applied), B = 16 keys from LDS;
//   online softmax per row (running max m, sum l; O rescaled by e^(m_old - m));
//   O += P V    v_mfma_f32_16x16x4_f32, A = P re-read from LDS, B = V from LDS.
// fp32 throughout, as the reference; results differ from the per-token
// softmax only in summation order.  Row stride padding makes the B reads of
// K (16 rows x 2 columns per half-wave: stride = 2 mod 32 banks), of V (2 rows x
// 16 columns: stride = 16 mod 32) and the A reads of P conflict-free.
// Outputs as the split/combine path: out rows (fp32) and their Q8_0 blocks.
// ---------------------------------------------------------------------------
typedef float v4f_t __attribute__((ext_vector_type(4)));

constexpr int kPfRows = 64;
constexpr int kPfKeys = 32;

template <int HD>
struct PfLayout {
    static constexpr int QS = HD + 4;        // Q tile row stride (floats)
    static constexpr int KS = HD + 2;        // K block row stride
    static constexpr int VS = HD + 16;       // V block row stride
    static constexpr int PS = kPfKeys + 2;   // P tile row stride
};

template <int HD>
__global__ __launch_bounds__(256) void k_attn_prefill(AttnArgs a, int G, int QT) {
    using Lay = PfLayout<HD>;
    constexpr int KSTEP = HD / 4;  // MFMA k-steps over the head dimension
    constexpr int DT = HD / 16;    // output column tiles
    constexpr int HALF = HD / 2;
    __shared__ __attribute__((aligned(16))) float qs[kPfRows * Lay::QS];
    __shared__ __attribute__((aligned(16))) float ks[kPfKeys * Lay::KS];
    __shared__ __attribute__((aligned(16))) float vs[kPfKeys * Lay::VS];
    __shared__ __attribute__((aligned(16))) float ps[4][16 * Lay::PS];

    const int kvh = blockIdx.x, qt0 = blockIdx.y * QT;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int pos0 = a.pos_dev ? *a.pos_dev : a.pos;
    const int n_tok = a.n_tok > 1 ? a.n_tok : 1;
    const int t_end = min(qt0 + QT, n_tok);  // tokens qt0 .. t_end-1
    const int kmax = pos0 + t_end - 1;       // last key any row attends to
    const size_t kve = (size_t)a.n_kv_heads * HD;

    // 1. Q tile: row r = token qt0 + r / G, head kvh*G + r % G (+ bias, RoPE)
    for (int idx = tid; idx < kPfRows * HD; idx += 256) {
        const int r = idx / HD, d = idx % HD, tl = r / G;
        float v = 0.f;
        if (tl < QT && qt0 + tl < n_tok) {
            const size_t e = (size_t)(kvh * G + r % G) * HD + d;
            v = a.q[(size_t)(qt0 + tl) * a.q_ld + e];
            if (a.bq) v += a.bq[e];
        }
        qs[r * Lay::QS + d] = v;
    }
    __syncthreads();
    if (a.cos_t) {
        for (int idx = tid; idx < kPfRows * HALF; idx += 256) {
            const int r = idx / HALF, i = idx % HALF, tl = r / G;
            if (tl < QT && qt0 + tl < n_tok) {
                const size_t pr = (size_t)(pos0 + qt0 + tl) * HALF + i;
                const float c = a.cos_t[pr], sn = a.sin_t[pr];
                float* h = qs + r * Lay::QS;
                const float x0 = h[i], x1 = h[i + HALF];
                h[i] = fmaf(x0, c, -(x1 * sn));
                h[i + HALF] = fmaf(x0, sn, x1 * c);
            }
        }
        __syncthreads();
    }
    float qa[KSTEP];
#pragma unroll
    for (int k = 0; k < KSTEP; k++) qa[k] = qs[(16 * wave + col) * Lay::QS + 4 * k + grp];

    // this lane's four result rows 4*grp + i of the wave's 16: their positions
    int qpos[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 16 * wave + 4 * grp + i, tl = r / G;
        qpos[i] = (tl < QT && qt0 + tl < n_tok) ? pos0 + qt0 + tl : -1;  // -1: no row
    }
    const float scale = 1.f / sqrtf((float)HD);
    float m[4], l[4];
    v4f_t o[DT];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        m[i] = -INFINITY;
        l[i] = 0.f;
    }
#pragma unroll
    for (int t = 0; t < DT; t++) o[t] = v4f_t{0.f, 0.f, 0.f, 0.f};

    // K/V blocks stream through registers: block kb+32 is loaded while block kb
    // is used from LDS.  Rows past kmax re-read row kmax (masked below).
    constexpr int NLD = kPfKeys * HD / 4 / 256;  // float4 of K (and of V) per thread
    float4 kreg[NLD], vreg[NLD];
    auto load_block = [&](int kb) {
#pragma unroll
        for (int u = 0; u < NLD; u++) {
            const int idx = tid + 256 * u, r = idx / (HD / 4), c4 = idx % (HD / 4);
            const size_t off = (size_t)min(kb + r, kmax) * kve + (size_t)kvh * HD + 4 * c4;
            kreg[u] = *reinterpret_cast<const float4*>(a.kcache + off);
            vreg[u] = *reinterpret_cast<const float4*>(a.vcache + off);
        }
    };
    load_block(0);
    for (int kb = 0; kb <= kmax; kb += kPfKeys) {
        // 2. this block into LDS, the next one into registers
#pragma unroll
        for (int u = 0; u < NLD; u++) {
            const int idx = tid + 256 * u, r = idx / (HD / 4), c4 = idx % (HD / 4);
            float2* kd = reinterpret_cast<float2*>(ks + r * Lay::KS + 4 * c4);
            kd[0] = make_float2(kreg[u].x, kreg[u].y);
            kd[1] = make_float2(kreg[u].z, kreg[u].w);
            *reinterpret_cast<float4*>(vs + r * Lay::VS + 4 * c4) = vreg[u];
        }
        __syncthreads();
        if (kb + kPfKeys <= kmax) load_block(kb + kPfKeys);

        // 3. S for 16 rows x 32 keys (two 16-key tiles)
        v4f_t sacc[2];
#pragma unroll
        for (int ct = 0; ct < 2; ct++) {
            sacc[ct] = v4f_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < KSTEP; k++)
                sacc[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                    qa[k], ks[(16 * ct + col) * Lay::KS + 4 * k + grp], sacc[ct], 0, 0, 0);
        }
        // 4. online softmax of the lane's rows (16 lanes per row group share them)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float sv[2];
            float bm = -INFINITY;
#pragma unroll
            for (int ct = 0; ct < 2; ct++) {
                const int key = kb + 16 * ct + col;
                sv[ct] = (qpos[i] >= 0 && key <= qpos[i]) ? sacc[ct][i] * scale : -INFINITY;
                bm = fmaxf(bm, sv[ct]);
            }
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) bm = fmaxf(bm, __shfl_xor(bm, off, 16));
            const float mn = fmaxf(m[i], bm);
            // a row with nothing to attend to yet keeps zero weights
            const float alpha = mn == -INFINITY ? 1.f : expf(m[i] - mn);
            float rs = 0.f;
#pragma unroll
            for (int ct = 0; ct < 2; ct++) {
                const float p = mn == -INFINITY ? 0.f : expf(sv[ct] - mn);
                ps[wave][(4 * grp + i) * Lay::PS + 16 * ct + col] = p;
                rs += p;
            }
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) rs += __shfl_xor(rs, off, 16);
            l[i] = fmaf(l[i], alpha, rs);
            m[i] = mn;
#pragma unroll
            for (int t = 0; t < DT; t++) o[t][i] *= alpha;
        }
        __syncthreads();
        // 5. O += P V
        float pa[kPfKeys / 4];
#pragma unroll
        for (int k = 0; k < kPfKeys / 4; k++) pa[k] = ps[wave][col * Lay::PS + 4 * k + grp];
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int k = 0; k < kPfKeys / 4; k++)
                o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                    pa[k], vs[(4 * k + grp) * Lay::VS + 16 * t + col], o[t], 0, 0, 0);
        __syncthreads();
    }

    // 6. normalise, write the rows (fp32, through the Q tile's LDS for the Q8_0 pass)
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float inv = l[i] > 0.f ? 1.f / l[i] : 0.f;
        const int r = 16 * wave + 4 * grp + i;
#pragma unroll
        for (int t = 0; t < DT; t++) qs[r * Lay::QS + 16 * t + col] = o[t][i] * inv;
    }
    __syncthreads();
    for (int idx = tid; idx < kPfRows * HD; idx += 256) {
        const int r = idx / HD, d = idx % HD, tl = r / G;
        if (tl < QT && qt0 + tl < n_tok)
            a.out[(size_t)(qt0 + tl) * a.out_ld + (size_t)(kvh * G + r % G) * HD + d] =
                qs[r * Lay::QS + d];
    }
    if (a.outq8) {
        // one 32-value block per 8 lanes, as q8_store4 expects
        for (int idx = tid; idx < kPfRows * HD / 4; idx += 256) {
            const int r = idx / (HD / 4), c4 = idx % (HD / 4), tl = r / G;
            const float4 v = *reinterpret_cast<const float4*>(qs + r * Lay::QS + 4 * c4);
            const bool ok = tl < QT && qt0 + tl < n_tok;
            const size_t e0 = (size_t)(qt0 + (ok ? tl : 0)) * a.out_ld +
                              (size_t)(kvh * G + r % G) * HD + 4 * c4;
            // the 8 lanes of a block are consecutive and share r: all store or none
            if (ok) q8_store4(a.outq8 + (e0 >> 5) * Q8_0_BYTES, c4 & 7, v);
        }
    }
}

// ---------------------------------------------------------------------------
// The same attention with the keys split over the workgroup's waves (head
// dimensions 64 and 128): a workgroup owns 16 query rows of one kv head (QT =
// 16 / G tokens x the G query heads that share it) and its 4 waves take the
// 16-key tiles kt = wave, wave + 4, ... of keys 0 .. (its last token's
// position), each with its own online softmax state (running max m, sum l, O),
// merged at the end in wave order through LDS.  Per tile, straight from the
// cache into registers (no LDS staging):
//   S^T = K Q^T   v_mfma_f32_16x16x4_f32, A = 16 keys (lane: key col, dims
//                 grp*HD/4 .. +HD/4, contiguous), B = the 16 query rows (same
//                 dims); result lane: keys 4*grp + r of query col;
//   O^T += V^T P^T  A = V (lane: keys 4*grp + r, dims col*HD/16 .. +HD/16),
//                 B = P as the S^T result lane holds it (no transpose);
//                 result lane: dims (4*grp + r)*HD/16 + dt of query col.
// So the max over a tile's 16 keys is 4 values in the lane and two shuffles;
// l stays per lane until the merge.  Four times the workgroups of the 64-row
// kernel, longest key ranges first.  fp32 throughout; results differ from the
// per-token softmax only in summation order.
// ---------------------------------------------------------------------------
constexpr int kPfKsRows = 16;
constexpr int kPfKsWaves = 4;

template <int HD>
__global__ __launch_bounds__(kPfKsWaves * 64) void k_attn_prefill_ks(AttnArgs a, int G, int QT) {
    constexpr int KQ = HD / 4;   // dims per lane group: the k-steps of S^T
    constexpr int DT = HD / 16;  // dims per lane of a V row: the output tiles
    constexpr int HALF = HD / 2;
    constexpr int QS = HD + 4;   // LDS row stride (Q tile, then the waves' O rows)
    constexpr int R = kPfKsRows, NW = kPfKsWaves;
    __shared__ __attribute__((aligned(16))) float qs[NW * R * QS];
    __shared__ float mm[NW][R], ll[NW][R];

    const int kvh = blockIdx.x;
    const int qt0 = (int)(gridDim.y - 1 - blockIdx.y) * QT;  // longest key ranges first
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, grp = lane >> 4;
    const int pos0 = a.pos_dev ? *a.pos_dev : a.pos;
    const int n_tok = a.n_tok > 1 ? a.n_tok : 1;
    const int t_end = min(qt0 + QT, n_tok);
    const int kmax = pos0 + t_end - 1;  // last key any row attends to
    const size_t kve = (size_t)a.n_kv_heads * HD;

    // 1. Q tile: row r = token qt0 + r / G, head kvh*G + r % G (+ bias, RoPE)
    for (int idx = tid; idx < R * HD; idx += NW * 64) {
        const int r = idx / HD, d = idx % HD, tl = r / G;
        float v = 0.f;
        if (tl < QT && qt0 + tl < n_tok) {
            const size_t e = (size_t)(kvh * G + r % G) * HD + d;
            v = a.q[(size_t)(qt0 + tl) * a.q_ld + e];
            if (a.bq) v += a.bq[e];
        }
        qs[r * QS + d] = v;
    }
    __syncthreads();
    if (a.cos_t) {
        for (int idx = tid; idx < R * HALF; idx += NW * 64) {
            const int r = idx / HALF, i = idx % HALF, tl = r / G;
            if (tl < QT && qt0 + tl < n_tok) {
                const size_t pr = (size_t)(pos0 + qt0 + tl) * HALF + i;
                const float c = a.cos_t[pr], sn = a.sin_t[pr];
                float* h = qs + r * QS;
                const float x0 = h[i], x1 = h[i + HALF];
                h[i] = fmaf(x0, c, -(x1 * sn));
                h[i + HALF] = fmaf(x0, sn, x1 * c);
            }
        }
        __syncthreads();
    }
    float qb[KQ];  // B operand of S^T: query col, dims grp*KQ + s
#pragma unroll
    for (int u = 0; u < KQ / 4; u++) {
        const float4 v = *reinterpret_cast<const float4*>(qs + col * QS + grp * KQ + 4 * u);
        qb[4 * u] = v.x; qb[4 * u + 1] = v.y; qb[4 * u + 2] = v.z; qb[4 * u + 3] = v.w;
    }
    const int qpos = (col / G < QT && qt0 + col / G < n_tok) ? pos0 + qt0 + col / G : -1;
    const float scale = 1.f / sqrtf((float)HD);

    float m = -INFINITY, l = 0.f;
    v4f_t o[DT];
#pragma unroll
    for (int t = 0; t < DT; t++) o[t] = v4f_t{0.f, 0.f, 0.f, 0.f};
    const float* kb = a.kcache + (size_t)kvh * HD;
    const float* vb = a.vcache + (size_t)kvh * HD;
    const int ntile = kmax / 16 + 1;
    // this lane's K row (key 16kt + col) and V rows (keys 16kt + 4grp + r), keys
    // past kmax re-read row kmax (masked below)
    float kr[KQ], vr[4][DT];
    auto load = [&](int kt) {
        const float4* kp = reinterpret_cast<const float4*>(
            kb + (size_t)min(16 * kt + col, kmax) * kve + grp * KQ);
#pragma unroll
        for (int u = 0; u < KQ / 4; u++) {
            const float4 v = kp[u];
            kr[4 * u] = v.x; kr[4 * u + 1] = v.y; kr[4 * u + 2] = v.z; kr[4 * u + 3] = v.w;
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float4* vp = reinterpret_cast<const float4*>(
                vb + (size_t)min(16 * kt + 4 * grp + r, kmax) * kve + col * DT);
#pragma unroll
            for (int u = 0; u < DT / 4; u++) {
                const float4 v = vp[u];
                vr[r][4 * u] = v.x; vr[r][4 * u + 1] = v.y; vr[r][4 * u + 2] = v.z; vr[r][4 * u + 3] = v.w;
            }
        }
    };
    // head dimension 64: the next tile's rows load during this one; 128: each
    // tile loads its own (the prefetch registers would leave two waves per SIMD
    // instead of three: 7B 512-token prefill 22.9 -> 22.7 ms without it, the
    // Qwen2.5-0.5B shape 5.36 -> 5.41 ms)
    constexpr bool PF = HD <= 64;
    if (PF && wave < ntile) load(wave);
    for (int kt = wave; kt < ntile; kt += NW) {
        float kc[KQ], vc[4][DT];
        if (!PF) load(kt);
#pragma unroll
        for (int s = 0; s < KQ; s++) kc[s] = kr[s];
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int t = 0; t < DT; t++) vc[r][t] = vr[r][t];
        if (PF && kt + NW < ntile) load(kt + NW);  // in flight during this tile
        v4f_t s4 = v4f_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KQ; s++) s4 = __builtin_amdgcn_mfma_f32_16x16x4f32(kc[s], qb[s], s4, 0, 0, 0);
        // online softmax of query col over keys 16kt + 4grp + r
        float sv[4], tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int key = 16 * kt + 4 * grp + r;
            sv[r] = (qpos >= 0 && key <= qpos) ? s4[r] * scale : -INFINITY;
            tmax = fmaxf(tmax, sv[r]);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float mn = fmaxf(m, tmax);
        // a row with nothing to attend to yet keeps zero weights
        const float alpha = mn == -INFINITY ? 1.f : expf(m - mn);
        float p[4], ps = 0.f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            p[r] = mn == -INFINITY ? 0.f : expf(sv[r] - mn);
            ps += p[r];
        }
        l = fmaf(l, alpha, ps);
        m = mn;
#pragma unroll
        for (int t = 0; t < DT; t++) {
            o[t] *= alpha;
#pragma unroll
            for (int r = 0; r < 4; r++) o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vc[r][t], p[r], o[t], 0, 0, 0);
        }
    }

    // 2. merge the waves' states (the Q tile is no longer read)
    __syncthreads();
    {
        float* ow = qs + (wave * R + col) * QS + grp * KQ;  // dims grp*KQ + r*DT + t
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int t4 = 0; t4 < DT / 4; t4++)
                *reinterpret_cast<float4*>(ow + r * DT + 4 * t4) =
                    make_float4(o[4 * t4][r], o[4 * t4 + 1][r], o[4 * t4 + 2][r], o[4 * t4 + 3][r]);
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        if (grp == 0) {
            mm[wave][col] = m;
            ll[wave][col] = l;
        }
    }
    __syncthreads();
    for (int idx = tid; idx < R * HD / 4; idx += NW * 64) {
        const int r = idx / (HD / 4), c4 = idx % (HD / 4), tl = r / G;
        float M = mm[0][r];
#pragma unroll
        for (int w = 1; w < NW; w++) M = fmaxf(M, mm[w][r]);
        float L = 0.f;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float f = mm[w][r] == -INFINITY ? 0.f : expf(mm[w][r] - M);
            L = fmaf(ll[w][r], f, L);
            v = fma4(f, *reinterpret_cast<const float4*>(qs + (w * R + r) * QS + 4 * c4), v);
        }
        const float inv = L > 0.f ? 1.f / L : 0.f;
        v = make_float4(v.x * inv, v.y * inv, v.z * inv, v.w * inv);
        // the 8 lanes of a Q8_0 block are consecutive and share r: all store or none
        if (tl < QT && qt0 + tl < n_tok) {
            const int t = qt0 + tl;
            const size_t e0 = (size_t)t * a.out_ld + (size_t)(kvh * G + r % G) * HD + 4 * c4;
            float* dst = a.out + e0;
            dst[0] = v.x;
            dst[1] = v.y;
            dst[2] = v.z;
            dst[3] = v.w;
            if (a.outq8) {
                const int sub = c4 & 7;
                float d;
                const uint32_t p = q8_quant4(v, d);  // q8_store4's block
                uint8_t* blk = a.outq8 + (e0 >> 5) * Q8_0_BYTES;
                *reinterpret_cast<uint32_t*>(blk + 4 + 4 * sub) = p;
                if (sub == 0) *reinterpret_cast<float*>(blk) = d;
                if (a.xh) {  // k_gemm_prep16's re-layout of the block (out_ld % 32 == 0)
                    const int kb = (int)((e0 - (size_t)t * a.out_ld) >> 5), Tp = a.Tp;
                    _Float16 hv[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) hv[e] = (_Float16)(float)(int8_t)(p >> (8 * e));
                    *reinterpret_cast<uint2*>(a.xh + (((size_t)kb * 4 + (sub >> 1)) * Tp + t) * 16 +
                                              (sub & 1) * 8) = *reinterpret_cast<const uint2*>(hv);
                    int sum = dot4((int)p, 0x01010101, 0);
                    sum += __shfl_xor(sum, 1, 8);
                    sum += __shfl_xor(sum, 2, 8);
                    sum += __shfl_xor(sum, 4, 8);
                    if (sub == 0) {
                        const size_t i2 = (((size_t)kb * (Tp / 32) + t / 32) * 16 + (t & 15)) * 2 + ((t >> 4) & 1);
                        const size_t i4 = (((size_t)kb * (Tp / 64) + t / 64) * 16 + (t & 15)) * 4 + ((t >> 4) & 3);
                        a.dx2[i2] = d;
                        a.gx2[i2] = d * (float)sum;
                        a.dx4[i4] = d;
                    }
                }
            }
        }
    }
}

int attn_nsplit(int max_seq) { return (max_seq + kAttnSplit - 1) / kAttnSplit; }

template <int HD>
static hipError_t launch_prefill_hd(const AttnArgs& a, int G, hipStream_t st) {
    const int nt = a.n_tok > 1 ? a.n_tok : 1;
    if constexpr (HD <= 128) {
        const int QT = kPfKsRows / G;
        const dim3 grid((unsigned)a.n_kv_heads, (unsigned)((nt + QT - 1) / QT));
        hipLaunchKernelGGL((k_attn_prefill_ks<HD>), grid, dim3(kPfKsWaves * 64), 0, st, a, G, QT);
        return hipGetLastError();
    }
    const int QT = kPfRows / G;
    const dim3 grid((unsigned)a.n_kv_heads, (unsigned)((nt + QT - 1) / QT));
    hipLaunchKernelGGL((k_attn_prefill<HD>), grid, dim3(256), 0, st, a, G, QT);
    return hipGetLastError();
}

hipError_t launch_attention_prefill(const AttnArgs& a, int head_dim, hipStream_t st) {
    if (a.n_kv_heads <= 0 || a.n_heads % a.n_kv_heads) return hipErrorInvalidValue;
    const int G = a.n_heads / a.n_kv_heads;
    if (G > 8 || a.store_kv || a.q_ld < a.n_heads * head_dim || a.out_ld < a.n_heads * head_dim ||
        (a.outq8 && a.out_ld % 32))
        return hipErrorInvalidValue;
    switch (head_dim) {
        case 64: return launch_prefill_hd<64>(a, G, st);
        case 128: return launch_prefill_hd<128>(a, G, st);
        case 256: return launch_prefill_hd<256>(a, G, st);
        default: return hipErrorInvalidValue;
    }
}

// Query heads per workgroup: all G of a kv head when kv heads x splits give
// `want` workgroups or more; fewer (down to 1) when they do not, so that a
// model with 2 kv heads of 8 query heads at context 1024 runs 136 workgroups
// of 2 heads instead of 34 of 8 (config-3 layer step 50.5 -> 43.0 us; 43.5 us
// with 272 workgroups of one head, 45.4 us with 68 of four).  Groups of one kv
// head each read its K/V rows (from L2 after the first).  want = 128, or 256
// at head dimension 64, where a workgroup's rows are half the bytes
// (Qwen2.5-0.5B shape, 2 kv heads of 7 at context 2048: 256 workgroups of 2
// heads instead of 128 of 4, decode step 789 -> 766 us).
static int attn_heads_per_group(int G, long kv_work, int hd) {
    const long want = hd == 64 ? 256 : 128;
    int gm = 1;
    while (gm < G && gm < 8) gm *= 2;  // G rounded up to a power of two
    while (gm > 1 && kv_work * ((G + gm - 1) / gm) < want) gm /= 2;
    return gm;
}

template <int HD>
static hipError_t launch_attn_hd(const AttnArgs& a, int G, hipStream_t st) {
    const unsigned nt = a.n_tok > 1 ? (unsigned)a.n_tok : 1u;
    const int gm = attn_heads_per_group(G, (long)a.n_kv_heads * a.nsplit * nt, HD);
    const dim3 grid((unsigned)(a.n_kv_heads * ((G + gm - 1) / gm)), (unsigned)a.nsplit, nt);
    if (gm == 1)
        hipLaunchKernelGGL((k_attn_split<HD, 1>), grid, dim3(kAttnThreads), 0, st, a);
    else if (gm == 2)
        hipLaunchKernelGGL((k_attn_split<HD, 2>), grid, dim3(kAttnThreads), 0, st, a);
    else if (gm == 4)
        hipLaunchKernelGGL((k_attn_split<HD, 4>), grid, dim3(kAttnThreads), 0, st, a);
    else if (gm == 8)
        hipLaunchKernelGGL((k_attn_split<HD, 8>), grid, dim3(kAttnThreads), 0, st, a);
    else
        return hipErrorInvalidValue;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_attn_combine<HD>), dim3((unsigned)a.n_heads, nt), dim3(kAttnThreads), 0,
                       st, a);
    return hipGetLastError();
}

hipError_t launch_qk_prep(const QkPrepArgs& a, int n_tok, hipStream_t st) {
    if (a.hd < 2 || a.hd > 256 || a.hd % 8 || n_tok < 1 || !a.cos_t || !a.sin_t ||
        (a.order != 1 && a.order != 2))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_qk_prep, dim3((unsigned)(a.n_heads + a.n_kv_heads), (unsigned)n_tok),
                       dim3(64), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_attention_fused(const AttnArgs& a, int head_dim, hipStream_t st) {
    if (a.n_kv_heads <= 0 || a.n_heads % a.n_kv_heads) return hipErrorInvalidValue;
    const int G = a.n_heads / a.n_kv_heads;
    if (a.nsplit < 1 || a.nsplit > kMaxSplit || G > 8 || (a.store_kv && !a.cos_t))
        return hipErrorInvalidValue;
    // several query rows: K/V rows already stored, row t at q + t*q_ld, out + t*out_ld
    if (a.n_tok > 1 && (a.store_kv || a.q_ld < a.n_heads * head_dim ||
                        a.out_ld < a.n_heads * head_dim || (a.outq8 && a.out_ld % 32)))
        return hipErrorInvalidValue;
    switch (head_dim) {
        case 64: return launch_attn_hd<64>(a, G, st);
        case 128: return launch_attn_hd<128>(a, G, st);
        case 256: return launch_attn_hd<256>(a, G, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace axf
