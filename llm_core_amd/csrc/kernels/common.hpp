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
// 16 bytes from a 2-byte aligned address: one global_load_dwordx4 (gfx9 global
// loads take unaligned addresses; a load that straddles a cache line costs a
// second line access, nothing else)
typedef uint32_t u32x4_a2_t __attribute__((ext_vector_type(4), aligned(2)));
__device__ __forceinline__ uint4 ld16_a2(const uint8_t* p) {
    const u32x4_a2_t v = *reinterpret_cast<const u32x4_a2_t*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
typedef uint32_t u32x2_a2_t __attribute__((ext_vector_type(2), aligned(2)));  // 8 bytes, 2-aligned

// Sum over groups of `width` consecutive lanes (width a power of two <= 64);
// every lane of the group receives the group sum.
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

// Sum over groups of `width` consecutive lanes (16, 32 or 64) with DPP row
// operations (no LDS round trips); the sum is valid in the LAST lane of each
// group.  quad_perm swaps, row_half_mirror and row_mirror reduce each 16-lane
// row; row_bcast:15 / row_bcast:31 carry row sums into rows 1, 3 and 2, 3.
template <int width>
__device__ __forceinline__ float group_sum_last(float v) {
    static_assert(width == 16 || width == 32 || width == 64, "DPP group width");
    v += __builtin_amdgcn_update_dpp(0.f, v, 0xb1, 0xf, 0xf, false);   // quad_perm 1,0,3,2
    v += __builtin_amdgcn_update_dpp(0.f, v, 0x4e, 0xf, 0xf, false);   // quad_perm 2,3,0,1
    v += __builtin_amdgcn_update_dpp(0.f, v, 0x141, 0xf, 0xf, false);  // row_half_mirror
    v += __builtin_amdgcn_update_dpp(0.f, v, 0x140, 0xf, 0xf, false);  // row_mirror
    if (width >= 32) v += __builtin_amdgcn_update_dpp(0.f, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
    if (width >= 64) v += __builtin_amdgcn_update_dpp(0.f, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return v;
}

// Reductions over groups of 8 consecutive lanes with DPP (quad_perm swaps,
// then row_half_mirror pairs each lane with one of the other quad); every
// lane of the group receives the result.  No LDS round trip (ds_bpermute).
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, __builtin_amdgcn_update_dpp(v, v, 0xb1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
    v = fmaxf(v, __builtin_amdgcn_update_dpp(v, v, 0x4e, 0xf, 0xf, false));   // quad_perm 2,3,0,1
    v = fmaxf(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xf, 0xf, false));  // row_half_mirror
    return v;
}
// Maximum over the 8-lane group of non-negative floats (absolute values),
// taken on their bit patterns: non-negative floats order as unsigned
// integers, so each DPP step is one integer max (fmaxf would add a
// canonicalisation per step).  Equals max8 for inputs that are not NaN.
__device__ __forceinline__ float max8_nonneg(float v) {
    uint32_t u = __float_as_uint(v);
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0xb1, 0xf, 0xf, false));
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x4e, 0xf, 0xf, false));
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x141, 0xf, 0xf, false));
    return __uint_as_float(u);
}
// sum over the lane's quad (every lane of the quad receives it)
__device__ __forceinline__ int sum_quad(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xb1, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x4e, 0xf, 0xf, false);
    return v;
}
// the value of lane 7 - (lane & 7) of the lane's group of 8 (row_half_mirror)
__device__ __forceinline__ int half_mirror(int v) {
    return __builtin_amdgcn_update_dpp(v, v, 0x141, 0xf, 0xf, false);
}

// Maximum over the wave, returned in every lane: the DPP steps of
// group_sum_last<64> with max (masked rows keep -inf), then lane 63 read into
// a scalar register.
__device__ __forceinline__ float wave_max_bcast(float v) {
    v = fmaxf(v, __builtin_amdgcn_update_dpp(-INFINITY, v, 0xb1, 0xf, 0xf, false));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(-INFINITY, v, 0x4e, 0xf, 0xf, false));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(-INFINITY, v, 0x141, 0xf, 0xf, false));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(-INFINITY, v, 0x140, 0xf, 0xf, false));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(-INFINITY, v, 0x142, 0xa, 0xf, false));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(-INFINITY, v, 0x143, 0xc, 0xf, false));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// SwiGLU of the reference (swiglu_avx2, llama_model.cpp:319-368): e = exp(-|g|)
// by the Cephes single-precision expf method (S. L. Moshier, Cephes Math
// Library: Cody-Waite reduction by ln2 in two constants, degree-5 polynomial,
// 2^n scaling), sigmoid = 1/(1+e) for g >= 0 and e/(1+e) for g < 0,
// out = (g*sigmoid)*up.
__device__ __forceinline__ float exp_cephes(float x) {
    float xx = fminf(x, 88.3762626648f);
    xx = fmaxf(-88.3762626648f, xx);
    const float fx = floorf(fmaf(xx, 1.44269504089f, 0.5f));
    xx = fmaf(-fx, 0.693359375f, xx);
    xx = fmaf(-fx, -2.12194440e-4f, xx);
    const float z = xx * xx;
    float p = 1.9875691500E-4f;
    p = fmaf(p, xx, 1.3981999507E-3f);
    p = fmaf(p, xx, 8.3334519073E-3f);
    p = fmaf(p, xx, 4.1665795894E-2f);
    p = fmaf(p, xx, 1.6666665459E-1f);
    p = fmaf(p, xx, 5.0000001201E-1f);
    p = fmaf(p, z, xx + 1.f);
    const int n = ((int)fx + 127) << 23;
    return p * __int_as_float(n);
}

__device__ __forceinline__ float swiglu1(float g, float u) {
    const float e = exp_cephes(-fabsf(g));
    const float denom = 1.f + e;
    const float sig = g < 0.f ? e / denom : 1.f / denom;
    return (g * sig) * u;
}

// Q8_0 of 32 values held by one thread (quantize_q8_avx2, quant_q8_avx2.cpp:33-84):
// d = amax/127, q = rint(v * 127/amax) saturated to int8, packed 4 per dword.
__device__ __forceinline__ void q8_quant32(const float (&v)[32], uint32_t (&q)[8], float& d) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    d = amax / 127.f;
    const float id = amax > 0.f ? 127.f / amax : 0.f;
    // 0 < amax < 127/FLT_MAX: id = +inf, every product +-inf or NaN, which the
    // reference's cvtps_epi32 turns into INT_MIN and its packs into -128
    const bool ovf = __builtin_isinf(id);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        uint32_t w = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float r = rintf(v[4 * k + j] * id);
            r = fminf(fmaxf(r, -128.f), 127.f);
            w |= ((uint32_t)((int)r & 0xff)) << (8 * j);
        }
        q[k] = ovf ? 0x80808080u : w;
    }
}

// RMS normalisation scale 1/sqrt(mean(x^2) + eps) over n floats (n % 4 == 0)
// with one fixed summation order, so every kernel that normalises the same x
// gets the same bits whatever its workgroup size: 1024 slots, slot s
// accumulating the squares of float4 s, s+1024, ... in ascending order (fmaf
// chain x, y, z, w); slots 64w..64w+63 reduced by the DPP row tree of
// group_sum_last into partial w; the 16 partials added in order.  Called by
// all NT threads of a workgroup (NT = 256, 512 or 1024) with the thread's
// float4s of x: xv[k] = float4 t + NT*k, zero past the end (thread t holds
// slots t + NT*j, j < 1024/NT).
// red: 16 floats of LDS.  Ends with a barrier.
template <int NT, int KPT>
__device__ __forceinline__ float rms_scale(const float4 (&xv)[KPT], int n, float eps, float* red) {
    constexpr int NS = 1024 / NT;
    static_assert(NS * NT == 1024, "workgroup of 256, 512 or 1024 threads");
    float s[NS];
#pragma unroll
    for (int j = 0; j < NS; j++) s[j] = 0.f;
#pragma unroll
    for (int k = 0; k < KPT; k++) {
        float& a = s[k % NS];
        a = fmaf(xv[k].x, xv[k].x, a);
        a = fmaf(xv[k].y, xv[k].y, a);
        a = fmaf(xv[k].z, xv[k].z, a);
        a = fmaf(xv[k].w, xv[k].w, a);
    }
#pragma unroll
    for (int j = 0; j < NS; j++) {
        const float v = group_sum_last<64>(s[j]);  // valid in lane 63
        if ((threadIdx.x & 63) == 63) red[(threadIdx.x >> 6) + (NT / 64) * j] = v;
    }
    __syncthreads();
    // one wave adds the partials and takes the square root; the others read
    // the scale after a second barrier (the same bits in every workgroup)
    if (threadIdx.x < 64) {
        float ss = red[0];
#pragma unroll
        for (int w = 1; w < 16; w++) ss += red[w];
        const float r = 1.f / sqrtf(ss / (float)n + eps);
        if (threadIdx.x == 0) red[0] = r;
    }
    __syncthreads();
    return red[0];
}

// amax / 127, correctly rounded, for every non-negative finite amax:
// q0 = amax * RN(1/127), r = amax - q0 * 127 (exact by fma), q0 + r * RN(1/127).
// Checked against the IEEE division on all 2^31 - 2^23 non-negative finite
// floats (the fma correction of a product by the rounded reciprocal,
// P. Markstein, "Computation of elementary functions on the IBM RISC
// System/6000 processor", IBM J. Res. Dev. 34(1), 1990).
__device__ __forceinline__ float div127(float a) {
    constexpr float y = 1.f / 127.f;
    const float q0 = a * y;
    const float r = __builtin_fmaf(-q0, 127.f, a);
    return __builtin_fmaf(r, y, q0);
}

// rint(a * b) of |a * b| < 2^22 as the low byte of a float's bits: the
// product is rounded to fp32 first (the empty asm keeps the compiler from
// fusing it into the add: one rounding of the exact product could land on
// the other side of a half), then adding 1.5 * 2^23 rounds it to an integer
// (to nearest, ties to even, as rintf) that occupies the low mantissa bits,
// two's complement around 0x4B400000.
__device__ __forceinline__ uint32_t rint_mul_bits(float a, float b) {
    float p = a * b;
    asm volatile("" : "+v"(p));
    return __float_as_uint(p + 12582912.f);
}

// Q8_0 of one 32-value block held as float4 by 8 consecutive lanes
// (sub = lane & 7): returns this lane's 4 packed int8 and, in d, the block scale.
// Same bits as q8_quant32 on the block (for inputs that are not NaN): for a
// finite id, |v * id| rounds to at most 127 (|v| <= amax), so the int8
// saturation never applies and rint_mul_bits' low byte is the int8 value; an
// infinite id (0 < amax < 127/FLT_MAX) gives -128 for every value, as the
// reference's cvtps_epi32 + packs.
__device__ __forceinline__ uint32_t q8_quant4(float4 v, float& d) {
    const float amax =
        max8_nonneg(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    d = div127(amax);
    const float id = amax > 0.f ? 127.f / amax : 0.f;
    const uint32_t b0 = rint_mul_bits(v.x, id), b1 = rint_mul_bits(v.y, id);
    const uint32_t b2 = rint_mul_bits(v.z, id), b3 = rint_mul_bits(v.w, id);
    // low bytes of b0..b3 -> bytes 0..3 (v_perm_b32 selectors: 0-3 the second
    // operand's bytes, 4-7 the first's, 0x0c zero)
    const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(b3, b2, 0x04000c0cu);
    return __builtin_isinf(id) ? 0x80808080u : (lo | hi);
}

// Q8_0 block (fp32 d + 32 int8) from 8 consecutive lanes' float4s (q8_quant4),
// written at blk by lane sub = 0..7 of the group.
__device__ __forceinline__ void q8_block_store(uint8_t* blk, int sub, float4 v) {
    float d;
    const uint32_t packed = q8_quant4(v, d);
    *reinterpret_cast<uint32_t*>(blk + 4 + 4 * sub) = packed;
    if (sub == 0) *reinterpret_cast<float*>(blk) = d;
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
