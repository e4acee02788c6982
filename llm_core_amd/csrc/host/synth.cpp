// synth.cpp — deterministic synthetic GGUF weights (host code).
//
// The reference reads real GGUF files produced by llama.cpp; there is no
// network here, so tests and benchmarks draw fp32 weights N(0, std) from a
// seed and quantize them to valid Q4_K / Q6_K super-blocks with the simple
// min/max quantizers below.  The quantizer only has to produce valid blocks:
// parity is always checked on identical bytes fed to both sides.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../capi_internal.hpp"

namespace {

inline uint64_t splitmix64(uint64_t x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}

// Standard normal pair for pair index p (Box-Muller on two 53-bit uniforms).
inline void normal_pair(uint64_t seed, uint64_t p, double& z0, double& z1) {
    const uint64_t a = splitmix64(seed ^ splitmix64(2 * p));
    const uint64_t b = splitmix64(seed ^ splitmix64(2 * p + 1));
    const double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);  // (0, 1]
    const double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);           // [0, 1)
    const double r = std::sqrt(-2.0 * std::log(u1));
    z0 = r * std::cos(2.0 * M_PI * u2);
    z1 = r * std::sin(2.0 * M_PI * u2);
}

void fill_normal(float* dst, int64_t begin, int64_t end, uint64_t seed, float mean, float sd) {
    int64_t i = begin;
    if (i & 1) {
        double z0, z1;
        normal_pair(seed, (uint64_t)(i >> 1), z0, z1);
        dst[i - begin] = (float)(mean + sd * z1);
        i++;
    }
    for (; i + 1 < end; i += 2) {
        double z0, z1;
        normal_pair(seed, (uint64_t)(i >> 1), z0, z1);
        dst[i - begin] = (float)(mean + sd * z0);
        dst[i + 1 - begin] = (float)(mean + sd * z1);
    }
    if (i < end) {
        double z0, z1;
        normal_pair(seed, (uint64_t)(i >> 1), z0, z1);
        dst[i - begin] = (float)(mean + sd * z0);
    }
}

// fp32 -> IEEE binary16 bits, round to nearest even (finite, normal-range inputs
// plus subnormals; overflow saturates to inf).
uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    x &= 0x7fffffffu;
    if (x >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (x > 0x7f800000u ? 0x200u : 0));
    if (x >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520 -> inf
    if (x < 0x38800000u) {                                      // subnormal half
        if (x < 0x33000000u) return (uint16_t)sign;
        const uint32_t m = (x & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int)(x >> 23);  // 14..24
        uint32_t h = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (h & 1))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((x >> 13) - (112u << 10));
    const uint32_t rem = x & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
    return (uint16_t)(sign | h);
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int s = 0;
            while (!(m & 0x400u)) {
                m <<= 1;
                s++;
            }
            bits = sign | ((uint32_t)(113 - s) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

inline int nearest(float v) { return (int)std::lrintf(v); }

// Q4_K: per 32-weight sub-block j, scale_j = (max - min)/15 and min_j = -min
// (min clamped to <= 0); d = max scale / 63, dmin = max min / 63 (fp16);
// 6-bit sc_j, m_j; q = round((x + dmin*m_j)/(d*sc_j)) in [0, 15].
void quantize_q4k_block(uint8_t* out, const float* x) {
    float scale[8], minv[8];
    for (int j = 0; j < 8; j++) {
        float lo = 0.f, hi = -INFINITY;
        for (int l = 0; l < 32; l++) {
            lo = std::min(lo, x[32 * j + l]);
            hi = std::max(hi, x[32 * j + l]);
        }
        scale[j] = (hi - lo) / 15.f;
        minv[j] = -lo;
    }
    const float max_scale = *std::max_element(scale, scale + 8);
    const float max_min = *std::max_element(minv, minv + 8);
    const uint16_t dh = f32_to_f16(max_scale / 63.f);
    const uint16_t dmh = f32_to_f16(max_min / 63.f);
    const float d = f16_to_f32(dh), dmin = f16_to_f32(dmh);
    uint8_t sc[8], m[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = (uint8_t)(d > 0.f ? std::clamp(nearest(scale[j] / d), 0, 63) : 0);
        m[j] = (uint8_t)(dmin > 0.f ? std::clamp(nearest(minv[j] / dmin), 0, 63) : 0);
    }
    std::memcpy(out, &dh, 2);
    std::memcpy(out + 2, &dmh, 2);
    uint8_t* s = out + 4;
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
    uint8_t q[256];
    for (int j = 0; j < 8; j++) {
        const float ds = d * (float)sc[j], ms = dmin * (float)m[j];
        for (int l = 0; l < 32; l++) {
            const float v = x[32 * j + l];
            q[32 * j + l] = (uint8_t)(ds > 0.f ? std::clamp(nearest((v + ms) / ds), 0, 15) : 0);
        }
    }
    uint8_t* qs = out + 16;
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++)
            qs[32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
}

// Q6_K: per 16-weight group g, scale_g = amax/31 (q in [-32, 31]); d = max
// scale / 127 (fp16); int8 sc_g; stored as q+32 split into ql/qh.
void quantize_q6k_block(uint8_t* out, const float* x) {
    float scale[16];
    for (int g = 0; g < 16; g++) {
        float amax = 0.f;
        for (int l = 0; l < 16; l++) amax = std::max(amax, std::fabs(x[16 * g + l]));
        scale[g] = amax / 31.f;
    }
    const float max_scale = *std::max_element(scale, scale + 16);
    const uint16_t dh = f32_to_f16(max_scale / 127.f);
    const float d = f16_to_f32(dh);
    int8_t sc[16];
    for (int g = 0; g < 16; g++) sc[g] = (int8_t)(d > 0.f ? std::clamp(nearest(scale[g] / d), 0, 127) : 0);
    uint8_t q[256];
    for (int i = 0; i < 256; i++) {
        const float s = d * (float)sc[i / 16];
        const int v = s > 0.f ? std::clamp(nearest(x[i] / s), -32, 31) : 0;
        q[i] = (uint8_t)(v + 32);
    }
    uint8_t* ql = out;
    uint8_t* qh = out + 128;
    std::memset(out, 0, 192);
    for (int n = 0; n < 2; n++) {
        for (int l = 0; l < 32; l++) {
            const uint8_t q1 = q[128 * n + l], q2 = q[128 * n + l + 32];
            const uint8_t q3 = q[128 * n + l + 64], q4 = q[128 * n + l + 96];
            ql[64 * n + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
            ql[64 * n + l + 32] = (uint8_t)((q2 & 15) | ((q4 & 15) << 4));
            qh[32 * n + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    }
    std::memcpy(out + 192, sc, 16);
    std::memcpy(out + 208, &dh, 2);
}

int block_bytes(int qtype) {
    return qtype == AXF_TYPE_Q4_K ? 144 : (qtype == AXF_TYPE_Q6_K ? 210 : 0);
}

template <class F>
void parallel_rows(int64_t n, F&& fn) {
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (n < 64) nt = 1;
    std::vector<std::thread> th;
    const int64_t chunk = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; t++) {
        const int64_t b = (int64_t)t * chunk, e = std::min(n, b + chunk);
        if (b >= e) break;
        th.emplace_back([&fn, b, e] { fn(b, e); });
    }
    for (auto& x : th) x.join();
}

}  // namespace

extern "C" {

int axf_synth_normal(float* dst, int64_t n, uint64_t seed, float mean, float stddev) {
    if (!dst || n < 0) return axf::fail(AXF_ERR_INVALID_ARG, "axf_synth_normal: bad arguments");
    parallel_rows((n + 4095) / 4096, [&](int64_t b, int64_t e) {
        const int64_t lo = b * 4096, hi = std::min(n, e * 4096);
        fill_normal(dst + lo, lo, hi, seed, mean, stddev);
    });
    return AXF_OK;
}

int axf_synth_quantize(int qtype, uint8_t* dst, const float* src, int64_t n) {
    if (!dst || !src || n < 0 || n % 256)
        return axf::fail(AXF_ERR_INVALID_ARG, "axf_synth_quantize: bad arguments");
    const int bb = block_bytes(qtype);
    if (!bb) return axf::fail(AXF_ERR_UNSUPPORTED, "axf_synth_quantize: qtype must be Q4_K or Q6_K");
    parallel_rows(n / 256, [&](int64_t b, int64_t e) {
        for (int64_t i = b; i < e; i++) {
            if (qtype == AXF_TYPE_Q4_K)
                quantize_q4k_block(dst + i * bb, src + i * 256);
            else
                quantize_q6k_block(dst + i * bb, src + i * 256);
        }
    });
    return AXF_OK;
}

int axf_synth_weight(int qtype, uint8_t* dst, int64_t rows, int64_t cols, uint64_t seed,
                     float stddev) {
    if (!dst || rows < 0 || cols <= 0 || cols % 256)
        return axf::fail(AXF_ERR_INVALID_ARG, "axf_synth_weight: bad arguments");
    const int bb = block_bytes(qtype);
    if (!bb) return axf::fail(AXF_ERR_UNSUPPORTED, "axf_synth_weight: qtype must be Q4_K or Q6_K");
    const int64_t nb = cols / 256;
    parallel_rows(rows, [&](int64_t b, int64_t e) {
        std::vector<float> row((size_t)cols);
        for (int64_t r = b; r < e; r++) {
            fill_normal(row.data(), r * cols, (r + 1) * cols, seed, 0.f, stddev);
            for (int64_t k = 0; k < nb; k++) {
                uint8_t* o = dst + (size_t)(r * nb + k) * bb;
                if (qtype == AXF_TYPE_Q4_K)
                    quantize_q4k_block(o, row.data() + 256 * k);
                else
                    quantize_q6k_block(o, row.data() + 256 * k);
            }
        }
    });
    return AXF_OK;
}

}  // extern "C"
