// common.hpp — device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../capi_internal.hpp"  // block sizes (Q4_K 144 B, Q6_K 210 B, Q8_0 36 B), launchers

namespace axf {

// IEEE binary16 bits -> binary32 (exact; v_cvt_f32_f16).
__device__ __forceinline__ float h2f(uint32_t bits16) {
    _Float16 h;
    uint16_t b = (uint16_t)bits16;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// Byte-aligned funnel shift: ((hi:lo) >> (8*nbytes))[31:0]  (v_alignbyte_b32).
__device__ __forceinline__ uint32_t alignbyte(uint32_t hi, uint32_t lo, uint32_t nbytes) {
    return __builtin_amdgcn_alignbyte(hi, lo, nbytes);
}

__device__ __forceinline__ int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

__device__ __forceinline__ uint4 ld16(const uint8_t* p) {  // 16-byte aligned
    return *reinterpret_cast<const uint4*>(p);
}
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) {  // 4-byte aligned
    return *reinterpret_cast<const uint32_t*>(p);
}
__device__ __forceinline__ uint32_t ld2(const uint8_t* p) {  // 2-byte aligned
    return *reinterpret_cast<const uint16_t*>(p);
}

// Sum over groups of `width` consecutive lanes (width a power of two <= 64);
// every lane of the group receives the group sum.
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// Q4_K scale/min pair for sub-blocks j0 = 2*part and j1 = 2*part + 1 from the
// 12 packed scale bytes s[0..11] held in three dwords (get_scale_min_k4 logic:
// j<4: sc=s[j]&63, m=s[j+4]&63;  j>=4: sc=(s[j+4]&15)|((s[j-4]>>6)<<4),
// m=(s[j+4]>>4)|((s[j]>>6)<<4)), evaluated bytewise and branch-free.
__device__ __forceinline__ void q4k_scales(uint32_t s03, uint32_t s47, uint32_t s811, int part,
                                           uint32_t& sc0, uint32_t& m0, uint32_t& sc1,
                                           uint32_t& m1) {
    const uint32_t sc_lo = s03 & 0x3f3f3f3fu;
    const uint32_t m_lo = s47 & 0x3f3f3f3fu;
    const uint32_t sc_hi = (s811 & 0x0f0f0f0fu) | ((s03 >> 2) & 0x30303030u);
    const uint32_t m_hi = ((s811 >> 4) & 0x0f0f0f0fu) | ((s47 >> 2) & 0x30303030u);
    const uint32_t scp = part < 2 ? sc_lo : sc_hi;
    const uint32_t mp = part < 2 ? m_lo : m_hi;
    const uint32_t sh = (part & 1) * 16;
    sc0 = (scp >> sh) & 0xffu;
    sc1 = (scp >> (sh + 8)) & 0xffu;
    m0 = (mp >> sh) & 0xffu;
    m1 = (mp >> (sh + 8)) & 0xffu;
}

}  // namespace axf
