// gemv.hip — fused-dequant GEMV for GGUF Q4_K / Q6_K weights on gfx950.
//
// y[o] = (accumulate ? y[o] : 0) + sum_k W[o,k] * x[k]   for o in [0, rows)
//
// Weights stay in the native GGUF super-block layout (rows contiguous,
// row_bytes apart).  Work decomposition (all four kernels):
//   * a "chunk" is 64 weights of one row: Q4_K chunk c = (block c/4, part c%4)
//     covers sub-blocks 2*part, 2*part+1 (qs bytes 32*part..+31, low and high
//     nibbles); Q6_K chunk c = (block c/4, half (c>>1)&1, t = c&1) covers the
//     32-weight parts s=t and s=t+2 of that half (they share their ql bytes).
//   * LPR lanes cooperate on a row (LPR = 16/32/64), each lane owns chunks
//     rl, rl+LPR, ... (CPL of them) for NR rows, so a wave covers
//     NR*64/LPR rows.  All weight loads of a lane are issued before the
//     activation is staged, which keeps NR*CPL*48 bytes per lane in flight.
//   * the activation is staged once per workgroup in LDS: for the Q8_0 kernels
//     as 80-byte per-chunk records (two 32-int8 Q8_0 blocks, their scales and
//     int sums; the 80-byte stride makes the ds_read_b128 of 16 consecutive
//     lanes hit 64 distinct banks), for the F32 kernels as padded float rows.
//   * the integer dot of a 32-weight Q8_0 block is exact (v_dot4_i32_i8);
//     fp32 scale products follow the reference kernels: (d*sc)*dx, (dmin*m)*dx.
//   * partial sums are reduced over the LPR lanes with cross-lane shuffles.
#include "common.hpp"

namespace axf {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

struct KernCfg {
    int lpr, cpl, nr;
};

static inline KernCfg pick_cfg(int nchunks) {
    KernCfg k;
    k.lpr = nchunks <= 16 ? 16 : (nchunks <= 32 ? 32 : 64);
    k.cpl = (nchunks + k.lpr - 1) / k.lpr;
    k.nr = k.cpl >= 4 ? 1 : (k.cpl == 3 ? 1 : 4 / k.cpl);
    return k;
}

// ---------------------------------------------------------------------------
// Activation staging
// ---------------------------------------------------------------------------

// Q4_K chunk record c: Q8_0 blocks 2c, 2c+1 -> {qs0[8 dw], qs1[8 dw], d0, d1, sum0, sum1}.
__device__ __forceinline__ void stage_q8_q4k(uint32_t* rec, const uint8_t* xq8, int nchunks) {
    for (int c = threadIdx.x; c < nchunks; c += kThreads) {
        uint32_t* r = rec + 20 * c;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint8_t* b = xq8 + (size_t)(2 * c + j) * Q8_0_BYTES;
            int s = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t q = ld4(b + 4 + 4 * k);
                r[8 * j + k] = q;
                s = dot4((int)q, 0x01010101, s);
            }
            r[16 + j] = ld4(b);
            r[18 + j] = (uint32_t)s;
        }
    }
}

// Q6_K chunk record c: Q8_0 blocks P1 = 2c-(c&1) and P1+2 -> {qs1[8 dw], qs2[8 dw], d1, d2, pad}.
__device__ __forceinline__ void stage_q8_q6k(uint32_t* rec, const uint8_t* xq8, int nchunks) {
    for (int c = threadIdx.x; c < nchunks; c += kThreads) {
        uint32_t* r = rec + 20 * c;
        const int p1 = 2 * c - (c & 1);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint8_t* b = xq8 + (size_t)(p1 + 2 * j) * Q8_0_BYTES;
#pragma unroll
            for (int k = 0; k < 8; k++) r[8 * j + k] = ld4(b + 4 + 4 * k);
            r[16 + j] = ld4(b);
        }
    }
}

// F32 activation, padded: element i at float index i + 4*(i >> shift).
template <int shift>
__device__ __forceinline__ void stage_f32(float* xs, const float* x, int K) {
    for (int i4 = threadIdx.x; i4 < K / 4; i4 += kThreads) {
        const float4 v = reinterpret_cast<const float4*>(x)[i4];
        const int i = 4 * i4;
        *reinterpret_cast<float4*>(xs + i + 4 * (i >> shift)) = v;
    }
}

// ---------------------------------------------------------------------------
// Q6_K byte fetch: 2-byte aligned sources read as aligned dwords + alignbyte.
// ---------------------------------------------------------------------------
template <int N>
__device__ __forceinline__ void load_u2(const uint8_t* p, uint32_t (&out)[N]) {
    // p is 2-byte aligned; reads [p & ~3, (p & ~3) + 4*(N+1)) which stays inside
    // the 210-byte block for the ql/qh fields (N = 8).
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint8_t* base = reinterpret_cast<const uint8_t*>(a & ~uintptr_t(3));
    const uint32_t sh = (uint32_t)(a & 3);
    uint32_t w[N + 1];
#pragma unroll
    for (int k = 0; k <= N; k++) w[k] = ld4(base + 4 * k);
#pragma unroll
    for (int k = 0; k < N; k++) out[k] = alignbyte(w[k + 1], w[k], sh);
}

// Scales (16 bytes at blk+192) and d (2 bytes at blk+208) without touching
// bytes past blk+210.
__device__ __forceinline__ void load_q6_tail(const uint8_t* blk, uint32_t (&sc)[4], uint32_t& dbits) {
    const uint8_t* p = blk + 192;
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint8_t* base = reinterpret_cast<const uint8_t*>(a & ~uintptr_t(3));
    const uint32_t sh = (uint32_t)(a & 3);
    uint32_t w[5];
#pragma unroll
    for (int k = 0; k < 4; k++) w[k] = ld4(base + 4 * k);
    if (sh) {
        w[4] = ld4(base + 16);  // bytes p+14..p+17: inside the block
        dbits = w[4] >> 16;
    } else {
        w[4] = 0;
        dbits = ld2(p + 16);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) sc[k] = alignbyte(w[k + 1], w[k], sh);
}

// ---------------------------------------------------------------------------
// Q4_K x Q8_0
// ---------------------------------------------------------------------------
template <int LPR, int CPL, int NR>
__global__ __launch_bounds__(kThreads) void k_gemv_q4k_q8(float* __restrict__ y,
                                                          const uint8_t* __restrict__ W,
                                                          const uint8_t* __restrict__ xq8,
                                                          int rows, int nb, long row_bytes,
                                                          int accumulate) {
    extern __shared__ uint4 smem[];
    uint32_t* rec = reinterpret_cast<uint32_t*>(smem);
    constexpr int RPP = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rl = lane % LPR, rg = lane / LPR;
    const int nchunks = 4 * nb;
    const long row0 = ((long)blockIdx.x * kWaves + wave) * (RPP * NR) + rg;

    uint4 hdr[NR][CPL], qa[NR][CPL], qb[NR][CPL];
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const long row = row0 + (long)n * RPP;
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const int c = rl + i * LPR;
            if (row < rows && c < nchunks) {
                const uint8_t* blk = W + row * row_bytes + (long)(c >> 2) * Q4K_BYTES;
                const int part = c & 3;
                hdr[n][i] = ld16(blk);
                qa[n][i] = ld16(blk + 16 + 32 * part);
                qb[n][i] = ld16(blk + 32 + 32 * part);
            } else {
                hdr[n][i] = make_uint4(0, 0, 0, 0);
                qa[n][i] = qb[n][i] = make_uint4(0, 0, 0, 0);
            }
        }
    }

    stage_q8_q4k(rec, xq8, nchunks);
    __syncthreads();

    float acc[NR];
#pragma unroll
    for (int n = 0; n < NR; n++) acc[n] = 0.f;

#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int c = rl + i * LPR;
        if (c < nchunks) {
            const uint4* r4 = reinterpret_cast<const uint4*>(rec + 20 * c);
            const uint4 xa0 = r4[0], xa1 = r4[1], xb0 = r4[2], xb1 = r4[3], meta = r4[4];
            const float dx0 = __uint_as_float(meta.x), dx1 = __uint_as_float(meta.y);
            const float sx0 = (float)(int)meta.z, sx1 = (float)(int)meta.w;
            const uint32_t xa[8] = {xa0.x, xa0.y, xa0.z, xa0.w, xa1.x, xa1.y, xa1.z, xa1.w};
            const uint32_t xb[8] = {xb0.x, xb0.y, xb0.z, xb0.w, xb1.x, xb1.y, xb1.z, xb1.w};
            const int part = c & 3;
#pragma unroll
            for (int n = 0; n < NR; n++) {
                const uint4 h = hdr[n][i];
                const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
                uint32_t sc0, m0, sc1, m1;
                q4k_scales(h.y, h.z, h.w, part, sc0, m0, sc1, m1);
                const uint32_t q[8] = {qa[n][i].x, qa[n][i].y, qa[n][i].z, qa[n][i].w,
                                       qb[n][i].x, qb[n][i].y, qb[n][i].z, qb[n][i].w};
                int dlo = 0, dhi = 0;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    dlo = dot4((int)(q[k] & 0x0f0f0f0fu), (int)xa[k], dlo);
                    dhi = dot4((int)((q[k] >> 4) & 0x0f0f0f0fu), (int)xb[k], dhi);
                }
                const float s0 = ((float)sc0 * d) * dx0, mm0 = ((float)m0 * dmin) * dx0;
                const float s1 = ((float)sc1 * d) * dx1, mm1 = ((float)m1 * dmin) * dx1;
                float a = acc[n];
                a = fmaf(s0, (float)dlo, a);
                a = fmaf(-mm0, sx0, a);
                a = fmaf(s1, (float)dhi, a);
                a = fmaf(-mm1, sx1, a);
                acc[n] = a;
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const float v = group_sum<LPR>(acc[n]);
        const long row = row0 + (long)n * RPP;
        if (rl == 0 && row < rows) y[row] = accumulate ? y[row] + v : v;
    }
}

// ---------------------------------------------------------------------------
// Q4_K x F32
// ---------------------------------------------------------------------------
template <int LPR, int CPL, int NR>
__global__ __launch_bounds__(kThreads) void k_gemv_q4k_f32(float* __restrict__ y,
                                                           const uint8_t* __restrict__ W,
                                                           const float* __restrict__ x, int rows,
                                                           int nb, long row_bytes,
                                                           int accumulate) {
    extern __shared__ uint4 smem[];
    float* xs = reinterpret_cast<float*>(smem);
    constexpr int RPP = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rl = lane % LPR, rg = lane / LPR;
    const int nchunks = 4 * nb;
    const long row0 = ((long)blockIdx.x * kWaves + wave) * (RPP * NR) + rg;

    uint4 hdr[NR][CPL], qa[NR][CPL], qb[NR][CPL];
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const long row = row0 + (long)n * RPP;
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const int c = rl + i * LPR;
            if (row < rows && c < nchunks) {
                const uint8_t* blk = W + row * row_bytes + (long)(c >> 2) * Q4K_BYTES;
                const int part = c & 3;
                hdr[n][i] = ld16(blk);
                qa[n][i] = ld16(blk + 16 + 32 * part);
                qb[n][i] = ld16(blk + 32 + 32 * part);
            } else {
                hdr[n][i] = make_uint4(0, 0, 0, 0);
                qa[n][i] = qb[n][i] = make_uint4(0, 0, 0, 0);
            }
        }
    }

    stage_f32<6>(xs, x, nb * QK_K);  // 64-float chunk c at float offset 68*c
    __syncthreads();

    float acc[NR];
#pragma unroll
    for (int n = 0; n < NR; n++) acc[n] = 0.f;

#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int c = rl + i * LPR;
        if (c < nchunks) {
            const float4* xc = reinterpret_cast<const float4*>(xs + 68 * c);
            const int part = c & 3;
            float ds[NR][2], ms[NR][2];
#pragma unroll
            for (int n = 0; n < NR; n++) {
                const uint4 h = hdr[n][i];
                const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
                uint32_t sc0, m0, sc1, m1;
                q4k_scales(h.y, h.z, h.w, part, sc0, m0, sc1, m1);
                ds[n][0] = d * (float)sc0;
                ms[n][0] = dmin * (float)m0;
                ds[n][1] = d * (float)sc1;
                ms[n][1] = dmin * (float)m1;
            }
#pragma unroll
            for (int hi = 0; hi < 2; hi++) {
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const float4 xv = xc[8 * hi + k];
#pragma unroll
                    for (int n = 0; n < NR; n++) {
                        const uint32_t qw = k < 4 ? (&qa[n][i].x)[k] : (&qb[n][i].x)[k - 4];
                        const uint32_t nib = hi ? ((qw >> 4) & 0x0f0f0f0fu) : (qw & 0x0f0f0f0fu);
                        const float dd = ds[n][hi], mm = -ms[n][hi];
                        float a = acc[n];
                        a = fmaf(fmaf(dd, (float)(nib & 0xffu), mm), xv.x, a);
                        a = fmaf(fmaf(dd, (float)((nib >> 8) & 0xffu), mm), xv.y, a);
                        a = fmaf(fmaf(dd, (float)((nib >> 16) & 0xffu), mm), xv.z, a);
                        a = fmaf(fmaf(dd, (float)(nib >> 24), mm), xv.w, a);
                        acc[n] = a;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const float v = group_sum<LPR>(acc[n]);
        const long row = row0 + (long)n * RPP;
        if (rl == 0 && row < rows) y[row] = accumulate ? y[row] + v : v;
    }
}

// ---------------------------------------------------------------------------
// Q6_K x Q8_0
// ---------------------------------------------------------------------------
struct Q6Chunk {
    uint32_t ql[8], qh[8], sc[4], dbits;
};

__device__ __forceinline__ void load_q6_chunk(const uint8_t* blk, int c, Q6Chunk& k) {
    const int h = (c >> 1) & 1, t = c & 1;
    load_u2<8>(blk + 64 * h + 32 * t, k.ql);
    load_u2<8>(blk + 128 + 32 * h, k.qh);
    load_q6_tail(blk, k.sc, k.dbits);
}

template <int LPR, int CPL, int NR>
__global__ __launch_bounds__(kThreads) void k_gemv_q6k_q8(float* __restrict__ y,
                                                          const uint8_t* __restrict__ W,
                                                          const uint8_t* __restrict__ xq8,
                                                          int rows, int nb, long row_bytes,
                                                          int accumulate) {
    extern __shared__ uint4 smem[];
    uint32_t* rec = reinterpret_cast<uint32_t*>(smem);
    constexpr int RPP = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rl = lane % LPR, rg = lane / LPR;
    const int nchunks = 4 * nb;
    const long row0 = ((long)blockIdx.x * kWaves + wave) * (RPP * NR) + rg;

    Q6Chunk wk[NR][CPL];
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const long row = row0 + (long)n * RPP;
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const int c = rl + i * LPR;
            if (row < rows && c < nchunks) {
                load_q6_chunk(W + row * row_bytes + (long)(c >> 2) * Q6K_BYTES, c, wk[n][i]);
            } else {
#pragma unroll
                for (int k = 0; k < 8; k++) wk[n][i].ql[k] = wk[n][i].qh[k] = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) wk[n][i].sc[k] = 0;
                wk[n][i].dbits = 0;
            }
        }
    }

    stage_q8_q6k(rec, xq8, nchunks);
    __syncthreads();

    float acc[NR];
#pragma unroll
    for (int n = 0; n < NR; n++) acc[n] = 0.f;

#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int c = rl + i * LPR;
        if (c < nchunks) {
            const uint4* r4 = reinterpret_cast<const uint4*>(rec + 20 * c);
            const uint4 xa0 = r4[0], xa1 = r4[1], xb0 = r4[2], xb1 = r4[3], meta = r4[4];
            const float dxa = __uint_as_float(meta.x), dxb = __uint_as_float(meta.y);
            const uint32_t xa[8] = {xa0.x, xa0.y, xa0.z, xa0.w, xa1.x, xa1.y, xa1.z, xa1.w};
            const uint32_t xb[8] = {xb0.x, xb0.y, xb0.z, xb0.w, xb1.x, xb1.y, xb1.z, xb1.w};
            const int h = (c >> 1) & 1, t = c & 1;
#pragma unroll
            for (int n = 0; n < NR; n++) {
                const Q6Chunk& k6 = wk[n][i];
                const float d = h2f(k6.dbits);
                const uint32_t sa = h ? k6.sc[2] : k6.sc[0], sb = h ? k6.sc[3] : k6.sc[1];
                const int sA0 = (int8_t)(sa >> (16 * t)), sA1 = (int8_t)(sa >> (16 * t + 8));
                const int sB0 = (int8_t)(sb >> (16 * t)), sB1 = (int8_t)(sb >> (16 * t + 8));
                int iA0 = 0, iA1 = 0, iB0 = 0, iB1 = 0;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const uint32_t l = k6.ql[k], hb = k6.qh[k];
                    const uint32_t qA = (l & 0x0f0f0f0fu) | (((hb >> (2 * t)) & 0x03030303u) << 4);
                    const uint32_t qB =
                        ((l >> 4) & 0x0f0f0f0fu) | (((hb >> (2 * t + 4)) & 0x03030303u) << 4);
                    // sum (q - 32) * x: -32 per byte is 0xE0 as int8
                    if (k < 4) {
                        iA0 = dot4((int)qA, (int)xa[k], iA0);
                        iA0 = dot4((int)0xE0E0E0E0u, (int)xa[k], iA0);
                        iB0 = dot4((int)qB, (int)xb[k], iB0);
                        iB0 = dot4((int)0xE0E0E0E0u, (int)xb[k], iB0);
                    } else {
                        iA1 = dot4((int)qA, (int)xa[k], iA1);
                        iA1 = dot4((int)0xE0E0E0E0u, (int)xa[k], iA1);
                        iB1 = dot4((int)qB, (int)xb[k], iB1);
                        iB1 = dot4((int)0xE0E0E0E0u, (int)xb[k], iB1);
                    }
                }
                float a = acc[n];
                a = fmaf((d * (float)sA0) * dxa, (float)iA0, a);
                a = fmaf((d * (float)sA1) * dxa, (float)iA1, a);
                a = fmaf((d * (float)sB0) * dxb, (float)iB0, a);
                a = fmaf((d * (float)sB1) * dxb, (float)iB1, a);
                acc[n] = a;
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const float v = group_sum<LPR>(acc[n]);
        const long row = row0 + (long)n * RPP;
        if (rl == 0 && row < rows) y[row] = accumulate ? y[row] + v : v;
    }
}

// ---------------------------------------------------------------------------
// Q6_K x F32
// ---------------------------------------------------------------------------
template <int LPR, int CPL, int NR>
__global__ __launch_bounds__(kThreads) void k_gemv_q6k_f32(float* __restrict__ y,
                                                           const uint8_t* __restrict__ W,
                                                           const float* __restrict__ x, int rows,
                                                           int nb, long row_bytes,
                                                           int accumulate) {
    extern __shared__ uint4 smem[];
    float* xs = reinterpret_cast<float*>(smem);
    constexpr int RPP = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rl = lane % LPR, rg = lane / LPR;
    const int nchunks = 4 * nb;
    const long row0 = ((long)blockIdx.x * kWaves + wave) * (RPP * NR) + rg;

    Q6Chunk wk[NR][CPL];
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const long row = row0 + (long)n * RPP;
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const int c = rl + i * LPR;
            if (row < rows && c < nchunks) {
                load_q6_chunk(W + row * row_bytes + (long)(c >> 2) * Q6K_BYTES, c, wk[n][i]);
            } else {
#pragma unroll
                for (int k = 0; k < 8; k++) wk[n][i].ql[k] = wk[n][i].qh[k] = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) wk[n][i].sc[k] = 0;
                wk[n][i].dbits = 0;
            }
        }
    }

    stage_f32<5>(xs, x, nb * QK_K);  // 32-float part p at float offset 36*p
    __syncthreads();

    float acc[NR];
#pragma unroll
    for (int n = 0; n < NR; n++) acc[n] = 0.f;

#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int c = rl + i * LPR;
        if (c < nchunks) {
            const int h = (c >> 1) & 1, t = c & 1;
            const int p1 = 2 * c - t;
            const float4* xA = reinterpret_cast<const float4*>(xs + 36 * p1);
            const float4* xB = reinterpret_cast<const float4*>(xs + 36 * (p1 + 2));
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float4 va = xA[k], vb = xB[k];
#pragma unroll
                for (int n = 0; n < NR; n++) {
                    const Q6Chunk& k6 = wk[n][i];
                    const float d = h2f(k6.dbits);
                    const uint32_t sa = h ? k6.sc[2] : k6.sc[0], sb = h ? k6.sc[3] : k6.sc[1];
                    const int sh = 16 * t + (k < 4 ? 0 : 8);
                    const float s_a = d * (float)(int)(int8_t)(sa >> sh);
                    const float s_b = d * (float)(int)(int8_t)(sb >> sh);
                    const float b_a = -(s_a * 32.f), b_b = -(s_b * 32.f);
                    const uint32_t l = k6.ql[k], hb = k6.qh[k];
                    const uint32_t qA = (l & 0x0f0f0f0fu) | (((hb >> (2 * t)) & 0x03030303u) << 4);
                    const uint32_t qB =
                        ((l >> 4) & 0x0f0f0f0fu) | (((hb >> (2 * t + 4)) & 0x03030303u) << 4);
                    float a = acc[n];
                    a = fmaf(fmaf(s_a, (float)(qA & 0xffu), b_a), va.x, a);
                    a = fmaf(fmaf(s_a, (float)((qA >> 8) & 0xffu), b_a), va.y, a);
                    a = fmaf(fmaf(s_a, (float)((qA >> 16) & 0xffu), b_a), va.z, a);
                    a = fmaf(fmaf(s_a, (float)(qA >> 24), b_a), va.w, a);
                    a = fmaf(fmaf(s_b, (float)(qB & 0xffu), b_b), vb.x, a);
                    a = fmaf(fmaf(s_b, (float)((qB >> 8) & 0xffu), b_b), vb.y, a);
                    a = fmaf(fmaf(s_b, (float)((qB >> 16) & 0xffu), b_b), vb.z, a);
                    a = fmaf(fmaf(s_b, (float)(qB >> 24), b_b), vb.w, a);
                    acc[n] = a;
                }
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const float v = group_sum<LPR>(acc[n]);
        const long row = row0 + (long)n * RPP;
        if (rl == 0 && row < rows) y[row] = accumulate ? y[row] + v : v;
    }
}

// ---------------------------------------------------------------------------
// Batched Q4_K x Q8_0 (small M): Y[t*rows + o] for a tile of TT tokens.
// Same lane decomposition as the GEMV; each lane decodes its weights once and
// reuses them for the TT tokens staged in LDS (TT records per chunk).
// ---------------------------------------------------------------------------
template <int LPR, int CPL, int NR, int TT>
__global__ __launch_bounds__(kThreads) void k_gemm_q4k_q8(float* __restrict__ Y,
                                                          const uint8_t* __restrict__ W,
                                                          const uint8_t* __restrict__ XQ8,
                                                          int rows, int nb, long row_bytes,
                                                          int t0, int nt) {
    extern __shared__ uint4 smem[];
    uint32_t* rec = reinterpret_cast<uint32_t*>(smem);
    constexpr int RPP = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rl = lane % LPR, rg = lane / LPR;
    const int nchunks = 4 * nb;
    const long row0 = ((long)blockIdx.x * kWaves + wave) * (RPP * NR) + rg;
    const size_t tok_bytes = (size_t)nb * 8 * Q8_0_BYTES;

    uint4 hdr[NR][CPL], qa[NR][CPL], qb[NR][CPL];
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const long row = row0 + (long)n * RPP;
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const int c = rl + i * LPR;
            if (row < rows && c < nchunks) {
                const uint8_t* blk = W + row * row_bytes + (long)(c >> 2) * Q4K_BYTES;
                const int part = c & 3;
                hdr[n][i] = ld16(blk);
                qa[n][i] = ld16(blk + 16 + 32 * part);
                qb[n][i] = ld16(blk + 32 + 32 * part);
            } else {
                hdr[n][i] = make_uint4(0, 0, 0, 0);
                qa[n][i] = qb[n][i] = make_uint4(0, 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TT; t++)
        if (t < nt) stage_q8_q4k(rec + (size_t)t * 20 * nchunks, XQ8 + (size_t)(t0 + t) * tok_bytes,
                                 nchunks);
    __syncthreads();

    float acc[NR][TT];
#pragma unroll
    for (int n = 0; n < NR; n++)
#pragma unroll
        for (int t = 0; t < TT; t++) acc[n][t] = 0.f;

#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int c = rl + i * LPR;
        if (c < nchunks) {
            const int part = c & 3;
#pragma unroll
            for (int n = 0; n < NR; n++) {
                const uint4 h = hdr[n][i];
                const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
                uint32_t sc0, m0, sc1, m1;
                q4k_scales(h.y, h.z, h.w, part, sc0, m0, sc1, m1);
                const float ds0 = (float)sc0 * d, ms0 = (float)m0 * dmin;
                const float ds1 = (float)sc1 * d, ms1 = (float)m1 * dmin;
                const uint32_t q[8] = {qa[n][i].x, qa[n][i].y, qa[n][i].z, qa[n][i].w,
                                       qb[n][i].x, qb[n][i].y, qb[n][i].z, qb[n][i].w};
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    if (t < nt) {
                        const uint4* r4 =
                            reinterpret_cast<const uint4*>(rec + ((size_t)t * nchunks + c) * 20);
                        const uint4 xa0 = r4[0], xa1 = r4[1], xb0 = r4[2], xb1 = r4[3],
                                    meta = r4[4];
                        const uint32_t xa[8] = {xa0.x, xa0.y, xa0.z, xa0.w,
                                                xa1.x, xa1.y, xa1.z, xa1.w};
                        const uint32_t xb[8] = {xb0.x, xb0.y, xb0.z, xb0.w,
                                                xb1.x, xb1.y, xb1.z, xb1.w};
                        int dlo = 0, dhi = 0;
#pragma unroll
                        for (int k = 0; k < 8; k++) {
                            dlo = dot4((int)(q[k] & 0x0f0f0f0fu), (int)xa[k], dlo);
                            dhi = dot4((int)((q[k] >> 4) & 0x0f0f0f0fu), (int)xb[k], dhi);
                        }
                        const float dx0 = __uint_as_float(meta.x), dx1 = __uint_as_float(meta.y);
                        float a = acc[n][t];
                        a = fmaf(ds0 * dx0, (float)dlo, a);
                        a = fmaf(-(ms0 * dx0), (float)(int)meta.z, a);
                        a = fmaf(ds1 * dx1, (float)dhi, a);
                        a = fmaf(-(ms1 * dx1), (float)(int)meta.w, a);
                        acc[n][t] = a;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const long row = row0 + (long)n * RPP;
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const float v = group_sum<LPR>(acc[n][t]);
            if (rl == 0 && row < rows && t < nt) Y[(size_t)(t0 + t) * rows + row] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------

template <int LPR, int CPL, int NR>
static hipError_t launch_cfg(GemvKind kind, float* y, const void* W, const void* x, int rows,
                             int nb, long row_bytes, int accumulate, hipStream_t st) {
    constexpr int rows_per_wg = kWaves * (64 / LPR) * NR;
    const dim3 grid((unsigned)((rows + rows_per_wg - 1) / rows_per_wg));
    const dim3 block(kThreads);
    const int nchunks = 4 * nb;
    const auto* Wb = static_cast<const uint8_t*>(W);
    switch (kind) {
        case GemvKind::Q4K_Q8:
            hipLaunchKernelGGL((k_gemv_q4k_q8<LPR, CPL, NR>), grid, block, (size_t)nchunks * 80, st,
                               y, Wb, static_cast<const uint8_t*>(x), rows, nb, row_bytes,
                               accumulate);
            break;
        case GemvKind::Q6K_Q8:
            hipLaunchKernelGGL((k_gemv_q6k_q8<LPR, CPL, NR>), grid, block, (size_t)nchunks * 80, st,
                               y, Wb, static_cast<const uint8_t*>(x), rows, nb, row_bytes,
                               accumulate);
            break;
        case GemvKind::Q4K_F32:
            hipLaunchKernelGGL((k_gemv_q4k_f32<LPR, CPL, NR>), grid, block,
                               (size_t)nb * QK_K * 4 * 17 / 16, st, y, Wb,
                               static_cast<const float*>(x), rows, nb, row_bytes, accumulate);
            break;
        case GemvKind::Q6K_F32:
            hipLaunchKernelGGL((k_gemv_q6k_f32<LPR, CPL, NR>), grid, block,
                               (size_t)nb * QK_K * 4 * 9 / 8, st, y, Wb,
                               static_cast<const float*>(x), rows, nb, row_bytes, accumulate);
            break;
    }
    return hipGetLastError();
}

// Largest K handled: 8 chunks per lane at 64 lanes -> kMaxBlocksPerRow = 128 super-blocks.
hipError_t launch_gemv(GemvKind kind, float* y, const void* W, const void* x, int rows, int nb,
                       long row_bytes, int accumulate, hipStream_t st) {
    const KernCfg k = pick_cfg(4 * nb);
#define AXF_GEMV_CASE(L, C, N)                                                                \
    if (k.lpr == L && k.cpl == C && k.nr == N)                                                \
        return launch_cfg<L, C, N>(kind, y, W, x, rows, nb, row_bytes, accumulate, st);
    AXF_GEMV_CASE(16, 1, 4)
    AXF_GEMV_CASE(32, 1, 4)
    AXF_GEMV_CASE(64, 1, 4)
    AXF_GEMV_CASE(64, 2, 2)
    AXF_GEMV_CASE(64, 3, 1)
    AXF_GEMV_CASE(64, 4, 1)
    AXF_GEMV_CASE(64, 5, 1)
    AXF_GEMV_CASE(64, 6, 1)
    AXF_GEMV_CASE(64, 7, 1)
    AXF_GEMV_CASE(64, 8, 1)
#undef AXF_GEMV_CASE
    return hipErrorInvalidValue;
}

}  // namespace axf

namespace axf {

template <int LPR, int CPL, int NR, int TT>
static hipError_t launch_gemm_cfg(float* Y, const void* W, const void* XQ8, int rows, int T,
                                  int nb, long row_bytes, hipStream_t st) {
    constexpr int rows_per_wg = kWaves * (64 / LPR) * NR;
    const dim3 grid((unsigned)((rows + rows_per_wg - 1) / rows_per_wg));
    const size_t lds = (size_t)TT * 4 * nb * 80;
    for (int t0 = 0; t0 < T; t0 += TT) {
        const int nt = T - t0 < TT ? T - t0 : TT;
        hipLaunchKernelGGL((k_gemm_q4k_q8<LPR, CPL, NR, TT>), grid, dim3(kThreads), lds, st, Y,
                           static_cast<const uint8_t*>(W), static_cast<const uint8_t*>(XQ8), rows,
                           nb, row_bytes, t0, nt);
    }
    return hipGetLastError();
}

template <int TT>
static hipError_t launch_gemm_tt(float* Y, const void* W, const void* XQ8, int rows, int T,
                                 int nb, long row_bytes, hipStream_t st) {
    const KernCfg k = pick_cfg(4 * nb);
#define AXF_GEMM_CASE(L, C, N)                                                             \
    if (k.lpr == L && k.cpl == C && k.nr == N)                                             \
        return launch_gemm_cfg<L, C, N, TT>(Y, W, XQ8, rows, T, nb, row_bytes, st);
    AXF_GEMM_CASE(16, 1, 4)
    AXF_GEMM_CASE(32, 1, 4)
    AXF_GEMM_CASE(64, 1, 4)
    AXF_GEMM_CASE(64, 2, 2)
    AXF_GEMM_CASE(64, 3, 1)
    AXF_GEMM_CASE(64, 4, 1)
    AXF_GEMM_CASE(64, 5, 1)
    AXF_GEMM_CASE(64, 6, 1)
    AXF_GEMM_CASE(64, 7, 1)
    AXF_GEMM_CASE(64, 8, 1)
#undef AXF_GEMM_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_gemm_q4k_q8(float* Y, const void* W, const void* XQ8, int rows, int T, int nb,
                              long row_bytes, hipStream_t st) {
    // token tile: as many tokens as fit 64 KiB of LDS records (80 B per chunk)
    const size_t per_tok = (size_t)4 * nb * 80;
    int tt = (int)(65536 / per_tok);
    if (T >= 8 && tt >= 8) return launch_gemm_tt<8>(Y, W, XQ8, rows, T, nb, row_bytes, st);
    if (T >= 4 && tt >= 4) return launch_gemm_tt<4>(Y, W, XQ8, rows, T, nb, row_bytes, st);
    if (T >= 2 && tt >= 2) return launch_gemm_tt<2>(Y, W, XQ8, rows, T, nb, row_bytes, st);
    return launch_gemm_tt<1>(Y, W, XQ8, rows, T, nb, row_bytes, st);
}

}  // namespace axf
