// sample.hip — the generation loop's token choice on the device: repetition
// penalty, temperature / top-k / top-p sampling and greedy argmax, as
// llama_generate_cpu_impl does it on the host (src/models/llama_model.cpp:
// sample :1466-1498, apply_rep_penalty :1595-1605).
//
//   1. k_rep_penalty: one thread walks the last `last_n` history tokens in
//      order, dividing positive logits by the penalty and multiplying the
//      others (a token seen twice is penalised twice, as in the reference).
//   2. k_topk_chunks: each workgroup scores a 4096-entry chunk of the
//      vocabulary (logit / temperature, a correctly rounded division), sorts
//      it in LDS (bitonic, 64-bit keys: order-preserving value bits, then the
//      complemented index, so equal values keep the lower index first) and
//      writes its best kc keys.
//   3. k_sample_pick: one workgroup sorts the candidates of all chunks the same
//      way (in LDS up to 16384 candidates; beyond, k_sample_pick_large sorts
//      them in place in global memory) and keeps the first k — the
//      reference's partial_sort prefix (its order among exactly equal scores is
//      unspecified; here lower index first) — then one thread runs the reference's sequential float
//      arithmetic: probs = exp(s - max), their sum in order, division, the
//      top-p cut and renormalisation, and the pick of the first i with
//      r < cumulative probability.  r is the step's uniform draw, precomputed on
//      the host from the reference's std::mt19937 stream.
// Greedy (temperature <= 0) is the same path with k = 1 on the raw logits:
// the first index of the maximum, std::max_element.
#include "common.hpp"

namespace axf {

namespace {

constexpr int kChunk = 4096;      // vocabulary entries per k_topk_chunks workgroup
constexpr int kPickMax = 16384;   // candidates k_sample_pick sorts at once
constexpr int kSortThreads = 1024;

__device__ __forceinline__ uint32_t ordered_bits(float v) {
    const uint32_t u = __float_as_uint(v);
    return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}

__device__ __forceinline__ float from_ordered(uint32_t o) {
    const uint32_t u = (o & 0x80000000u) ? (o ^ 0x80000000u) : ~o;
    return __uint_as_float(u);
}

__device__ __forceinline__ uint64_t make_key(float v, int idx) {
    return ((uint64_t)ordered_bits(v) << 32) | (uint64_t)(~(uint32_t)idx);
}

// Sort N keys in LDS in descending order (N a power of two), all threads.
template <int N>
__device__ void bitonic_desc(uint64_t* k) {
    for (int size = 2; size <= N; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < N / 2; t += blockDim.x) {
                const int i = 2 * stride * (t / stride) + (t % stride);
                const int j = i + stride;
                const uint64_t a = k[i], b = k[j];
                // blocks with (i & size) == 0 sort descending, the others ascending
                const bool desc = (i & size) == 0;
                if (desc ? (a < b) : (a > b)) {
                    k[i] = b;
                    k[j] = a;
                }
            }
            __syncthreads();
        }
    }
}

__global__ __launch_bounds__(1) void k_rep_penalty(float* __restrict__ logits,
                                                   const int* __restrict__ hist,
                                                   const int* __restrict__ hist_n, int last_n,
                                                   float penalty, int n_vocab) {
    const int n = *hist_n;
    const int win = last_n < n ? last_n : n;
    for (int i = n - win; i < n; i++) {
        const int id = hist[i];
        if (id < 0 || id >= n_vocab) continue;
        const float v = logits[id];
        logits[id] = v > 0.f ? v / penalty : v * penalty;
    }
}

// inv_temp_div: divide by temperature (sampling) or take the raw logit (greedy)
__global__ __launch_bounds__(kSortThreads) void k_topk_chunks(uint64_t* __restrict__ cand,
                                                              const float* __restrict__ logits,
                                                              int n_vocab, float temperature,
                                                              int divide, int kc) {
    __shared__ uint64_t keys[kChunk];
    const int base = blockIdx.x * kChunk;
    for (int t = threadIdx.x; t < kChunk; t += kSortThreads) {
        const int i = base + t;
        uint64_t key = 0;  // below every real key
        if (i < n_vocab) {
            const float s = divide ? logits[i] / temperature : logits[i];
            key = make_key(s, i);
        }
        keys[t] = key;
    }
    __syncthreads();
    bitonic_desc<kChunk>(keys);
    for (int t = threadIdx.x; t < kc; t += kSortThreads) cand[(size_t)blockIdx.x * kc + t] = keys[t];
}

template <int N>
__device__ void pick_sorted(uint64_t* keys, const uint64_t* __restrict__ cand, int n_cand) {
    for (int t = threadIdx.x; t < N; t += kSortThreads) keys[t] = t < n_cand ? cand[t] : 0;
    __syncthreads();
    bitonic_desc<N>(keys);
}

// Final choice over keys sorted in descending order (one thread).  Outputs as
// the greedy argmax kernel: *out, and when given tokens[*step] = token,
// *step += 1, *pos += 1; the token is always appended to the penalty history
// (hist[*hist_n], *hist_n += 1) when hist is given.
__device__ void finish_pick(const uint64_t* keys, int k, float top_p,
                            const float* __restrict__ r_table, float r_fixed, int* out,
                            int* tokens, int* step, int* pos, int* hist, int* hist_n) {
    int chosen;
    if (k == 1) {
        chosen = (int)~(uint32_t)keys[0];
    } else {
        // probs[i] = exp(s_i - max), sum in order, normalise (llama_model.cpp:1478-1480);
        // the probabilities are recomputed on the fly instead of stored
        const float mx = from_ordered((uint32_t)(keys[0] >> 32));
        float sum = 0.f;
        for (int i = 0; i < k; i++) sum += expf(from_ordered((uint32_t)(keys[i] >> 32)) - mx);
        int kk = k;
        float sum2 = sum;  // the divisor of the final probabilities
        bool renorm = false;
        if (top_p < 1.0f) {  // nucleus cut (:1483-1490)
            float cum = 0.f;
            int cut = k;
            for (int i = 0; i < k; i++) {
                cum += expf(from_ordered((uint32_t)(keys[i] >> 32)) - mx) / sum;
                if (cum >= top_p) {
                    cut = i + 1;
                    break;
                }
            }
            sum2 = 0.f;
            for (int i = 0; i < cut; i++)
                sum2 += expf(from_ordered((uint32_t)(keys[i] >> 32)) - mx) / sum;
            kk = cut;
            renorm = true;
        }
        const float r = r_table ? r_table[step ? *step : 0] : r_fixed;
        float cum = 0.f;
        chosen = (int)~(uint32_t)keys[kk - 1];
        for (int i = 0; i < kk; i++) {
            float p = expf(from_ordered((uint32_t)(keys[i] >> 32)) - mx) / sum;
            if (renorm) p = p / sum2;
            cum += p;
            if (r < cum) {
                chosen = (int)~(uint32_t)keys[i];
                break;
            }
        }
    }
    *out = chosen;
    if (tokens && step) {
        tokens[*step] = chosen;
        *step += 1;
    }
    if (pos) *pos += 1;
    if (hist && hist_n) {
        hist[*hist_n] = chosen;
        *hist_n += 1;
    }
}

__global__ __launch_bounds__(kSortThreads) void k_sample_pick(
    int* __restrict__ out, const uint64_t* __restrict__ cand, int n_cand, int pow2, int k,
    float top_p, const float* __restrict__ r_table, float r_fixed, int* tokens, int* step,
    int* pos, int* hist, int* hist_n) {
    __shared__ uint64_t keys[kPickMax];
    switch (pow2) {
    case 1024: pick_sorted<1024>(keys, cand, n_cand); break;
    case 2048: pick_sorted<2048>(keys, cand, n_cand); break;
    case 4096: pick_sorted<4096>(keys, cand, n_cand); break;
    case 8192: pick_sorted<8192>(keys, cand, n_cand); break;
    default: pick_sorted<16384>(keys, cand, n_cand); break;
    }
    if (threadIdx.x == 0)
        finish_pick(keys, k, top_p, r_table, r_fixed, out, tokens, step, pos, hist, hist_n);
}

// More than kPickMax candidates (large top_k, or the whole of a large
// vocabulary): the workgroup pads them with zero keys to pow2 and sorts them in
// place in `cand` (bitonic, the same comparisons as bitonic_desc, global
// memory ordered between the workgroup's steps by the barriers), then the same
// final pass.  One workgroup: slow (a few ms at 2^18 keys) but any k works.
__global__ __launch_bounds__(kSortThreads) void k_sample_pick_large(
    int* __restrict__ out, uint64_t* __restrict__ cand, int n_cand, int pow2, int k, float top_p,
    const float* __restrict__ r_table, float r_fixed, int* tokens, int* step, int* pos, int* hist,
    int* hist_n) {
    for (int t = n_cand + (int)threadIdx.x; t < pow2; t += kSortThreads) cand[t] = 0;
    __syncthreads();
    for (int size = 2; size <= pow2; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < pow2 / 2; t += kSortThreads) {
                const int i = 2 * stride * (t / stride) + (t % stride);
                const int j = i + stride;
                const uint64_t a = cand[i], b = cand[j];
                const bool desc = (i & size) == 0;
                if (desc ? (a < b) : (a > b)) {
                    cand[i] = b;
                    cand[j] = a;
                }
            }
            __syncthreads();
        }
    }
    if (threadIdx.x == 0)
        finish_pick(cand, k, top_p, r_table, r_fixed, out, tokens, step, pos, hist, hist_n);
}

}  // namespace

int sample_chunks(int n_vocab) { return (n_vocab + kChunk - 1) / kChunk; }

// candidate keys the chunk pass writes
static long sample_n_cand(int n_vocab, int k) {
    const int kc = k < kChunk ? k : kChunk;
    return (long)sample_chunks(n_vocab) * kc;
}

// keys of `cand` launch_sample needs: the candidates, or beyond kPickMax the
// power of two the in-place sort pads them to
int sample_candidates(int n_vocab, int k) {
    const long n = sample_n_cand(n_vocab, k);
    if (n <= kPickMax) return (int)n;
    long p = kPickMax;
    while (p < n) p <<= 1;
    return p <= (1L << 30) ? (int)p : 0;
}

hipError_t launch_rep_penalty(float* logits, const int* hist, const int* hist_n, int last_n,
                              float penalty, int n_vocab, hipStream_t st) {
    hipLaunchKernelGGL(k_rep_penalty, dim3(1), dim3(1), 0, st, logits, hist, hist_n, last_n,
                       penalty, n_vocab);
    return hipGetLastError();
}

hipError_t launch_sample(int* out, uint64_t* cand, const float* logits, int n_vocab,
                         float temperature, int top_k, float top_p, const float* r_table,
                         float r_fixed, int* tokens, int* step, int* pos, int* hist, int* hist_n,
                         hipStream_t st) {
    const bool greedy = !(temperature > 0.f);
    int k = greedy ? 1 : ((top_k > 0 && top_k < n_vocab) ? top_k : n_vocab);
    const int kc = k < kChunk ? k : kChunk;
    const int chunks = sample_chunks(n_vocab);
    const int n_cand = (int)sample_n_cand(n_vocab, k);
    if (sample_candidates(n_vocab, k) == 0) return hipErrorInvalidValue;
    int pow2 = 1024;
    while (pow2 < n_cand) pow2 <<= 1;
    hipLaunchKernelGGL(k_topk_chunks, dim3(chunks), dim3(kSortThreads), 0, st, cand, logits,
                       n_vocab, temperature, greedy ? 0 : 1, kc);
    if (n_cand <= kPickMax)
        hipLaunchKernelGGL(k_sample_pick, dim3(1), dim3(kSortThreads), 0, st, out, cand, n_cand,
                           pow2, k, greedy ? 1.0f : top_p, r_table, r_fixed, tokens, step, pos,
                           hist, hist_n);
    else
        hipLaunchKernelGGL(k_sample_pick_large, dim3(1), dim3(kSortThreads), 0, st, out, cand,
                           n_cand, pow2, k, greedy ? 1.0f : top_p, r_table, r_fixed, tokens, step,
                           pos, hist, hist_n);
    return hipGetLastError();
}

}  // namespace axf
