// sampling.cpp — the host half of sampled generation: the reference's random
// stream and the kernel-level sampling entry point.
//
// llama_generate_cpu_impl seeds std::mt19937 rng(42) per call and draws one
// std::uniform_real_distribution<float>(0, 1) value per sample() call when the
// temperature is positive (src/models/llama_model.cpp:1556, :1494).  The
// draws do not depend on the logits, so the whole stream of a generation is
// computed here before decoding and read by the device sampler step by step.
//   * MT19937: Matsumoto & Nishimura's generator as C++ [rand.eng.mers] fixes
//     it (w=32, n=624, m=397, r=31, a=0x9908b0df, u=11, d=0xffffffff, s=7,
//     b=0x9d2c5680, t=15, c=0xefc60000, l=18, f=1812433253).
//   * The float draw of libstdc++'s uniform_real_distribution<float>:
//     generate_canonical<float, 24> with one 32-bit output, u / 2^32 in float
//     (u rounded to float first), a result of 1 replaced by the largest float
//     below 1; then (b - a) * x + a = x for [0, 1).
#include <cstring>
#include <vector>

#include "../capi_internal.hpp"

using namespace axf;

namespace {

struct Mt19937 {
    uint32_t mt[624];
    int idx = 624;

    explicit Mt19937(uint32_t seed) {
        mt[0] = seed;
        for (int i = 1; i < 624; i++) mt[i] = 1812433253u * (mt[i - 1] ^ (mt[i - 1] >> 30)) + (uint32_t)i;
    }
    void twist() {
        for (int i = 0; i < 624; i++) {
            const uint32_t y = (mt[i] & 0x80000000u) | (mt[(i + 1) % 624] & 0x7fffffffu);
            mt[i] = mt[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
        }
        idx = 0;
    }
    uint32_t next() {
        if (idx >= 624) twist();
        uint32_t y = mt[idx++];
        y ^= y >> 11;
        y ^= (y << 7) & 0x9d2c5680u;
        y ^= (y << 15) & 0xefc60000u;
        y ^= y >> 18;
        return y;
    }
};

float canonical_float(uint32_t u) {
    const float x = (float)u / 4294967296.0f;
    return x >= 1.0f ? 0x1.fffffep-1f : x;
}

}  // namespace

namespace axf {
void sampling_uniforms(uint32_t seed, float* out, int n) {
    Mt19937 g(seed);
    for (int i = 0; i < n; i++) out[i] = canonical_float(g.next());
}
}  // namespace axf

extern "C" {

int axf_mt19937(uint32_t seed, uint32_t* out, int n) {
    if (n < 0 || (n && !out)) return fail(AXF_ERR_INVALID_ARG, "axf_mt19937: bad arguments");
    Mt19937 g(seed);
    for (int i = 0; i < n; i++) out[i] = g.next();
    return AXF_OK;
}

int axf_sampling_uniforms(uint32_t seed, float* out, int n) {
    if (n < 0 || (n && !out)) return fail(AXF_ERR_INVALID_ARG, "axf_sampling_uniforms: bad arguments");
    sampling_uniforms(seed, out, n);
    return AXF_OK;
}

}  // extern "C"
