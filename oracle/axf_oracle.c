/*
 * axf_oracle.c — CPU parity oracle (TEST INFRASTRUCTURE ONLY, see axf_oracle.h).
 *
 * Reference: songqiuyu/llm_core, paths relative to the reference root.
 * Lane conventions: an AVX2 __m256 is restated as float[8]; "hsum8" is the
 * reference's hsum256_* (lo+hi, hadd, hadd), e.g. gemv_q4k_avx2.cpp:53-60.
 */
#include "axf_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* scalar primitives                                                        */
/* ------------------------------------------------------------------------ */

/* IEEE binary16 -> binary32, exact (F16C vcvtph2ps semantics; the reference
 * uses _mm_cvtph_ps in every kernel, e.g. gemv_q4k_avx2.cpp:46-48, and the
 * scalar f16_to_f32 at llama_model.cpp:101-121). */
float orc_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else { /* subnormal: renormalise */
            int shift = 0;
            while (!(m & 0x400u)) {
                m <<= 1;
                shift++;
            }
            m &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 + 1 - shift) << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13) | (m ? 0x00400000u : 0u); /* quiet NaN */
    } else {
        bits = sign | ((e + 127 - 15) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline uint16_t rd16(const uint8_t* p) {
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
}

/* get_scale_min_k4: llama_model.cpp:464-473, gemv_q4k_avx2.cpp:34-43. */
void orc_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* Horizontal sum of an 8-lane vector in the reference's order
 * (hsum256_, gemv_q4k_avx2.cpp:53-60): lo = v[0..3] + v[4..7]; two hadds. */
static inline float hsum8(const float v[8]) {
    float l0 = v[0] + v[4], l1 = v[1] + v[5], l2 = v[2] + v[6], l3 = v[3] + v[7];
    return (l0 + l1) + (l2 + l3);
}

/* ------------------------------------------------------------------------ */
/* dequantisation                                                           */
/* ------------------------------------------------------------------------ */

/* Q4_K row dequant: the Q4_K branch of emb_lookup, llama_model.cpp:899-928.
 * GCC 11 (-O3 -mfma, the reference's flags) contracts `d1*q - mf1` into a
 * single vfmsub, which is also what gemv_q4k_avx2.cpp:108-117 does with
 * _mm256_fmsub_ps; hence fmaf(d1, q, -mf1) with d1 = d*sc and mf1 = dmin*m
 * each rounded first. */
void orc_dequant_q4k(float* out, const uint8_t* blocks, int64_t nblocks) {
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = blocks + (size_t)b * ORC_Q4K_BYTES;
        const float d = orc_fp16_to_fp32(rd16(blk));
        const float dmin = orc_fp16_to_fp32(rd16(blk + 2));
        const uint8_t* scales = blk + 4;
        const uint8_t* qs = blk + 16;
        float* ob = out + (size_t)b * ORC_QK_K;
        for (int c = 0; c < 4; c++) {
            uint8_t sc1, m1, sc2, m2;
            orc_get_scale_min_k4(2 * c, scales, &sc1, &m1);
            orc_get_scale_min_k4(2 * c + 1, scales, &sc2, &m2);
            const float d1 = d * (float)sc1, mf1 = dmin * (float)m1;
            const float d2 = d * (float)sc2, mf2 = dmin * (float)m2;
            const uint8_t* q = qs + 32 * c;
            for (int l = 0; l < 32; l++) {
                ob[64 * c + l] = fmaf(d1, (float)(q[l] & 0x0f), -mf1);
                ob[64 * c + l + 32] = fmaf(d2, (float)(q[l] >> 4), -mf2);
            }
        }
    }
}

/* Q6_K row dequant: q6k_row_to_f32, llama_model.cpp:560-592;
 * y = (d*sc)*q with q = raw6 - 32 (two roundings, no contraction possible). */
void orc_dequant_q6k(float* out, const uint8_t* blocks, int64_t nblocks) {
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = blocks + (size_t)b * ORC_Q6K_BYTES;
        const float d = orc_fp16_to_fp32(rd16(blk + 208));
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* sc = (const int8_t*)(blk + 192);
        float* y = out + (size_t)b * ORC_QK_K;
        for (int n = 0; n < 2; n++) {
            for (int l = 0; l < 32; l++) {
                const int is = l / 16;
                const int q1 = ((ql[l] & 0x0f) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = ((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l + 0] = d * (float)sc[is + 0] * (float)q1;
                y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                y[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
            ql += 64;
            qh += 32;
            sc += 8;
            y += 128;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* F32-activation GEMV                                                      */
/* ------------------------------------------------------------------------ */

/* One row of gemv_q4k_avx2_range (gemv_q4k_avx2.cpp:72-130; the 4-row tile
 * :135-225 performs the same per-row operation sequence).  Two 8-lane
 * accumulators; weight = fmsub(d*sc, q, dmin*m); acc = fmadd(w, x, acc). */
static float q4k_f32_row(const uint8_t* row, const float* x, int in_dim) {
    float a0[8] = {0}, a1[8] = {0};
    const int nb = in_dim / ORC_QK_K;
    for (int b = 0; b < nb; b++) {
        const uint8_t* blk = row + (size_t)b * ORC_Q4K_BYTES;
        const float d = orc_fp16_to_fp32(rd16(blk));
        const float dmin = orc_fp16_to_fp32(rd16(blk + 2));
        float ds[8], ms[8];
        for (int j = 0; j < 8; j++) {
            uint8_t sc, mn;
            orc_get_scale_min_k4(j, blk + 4, &sc, &mn);
            ds[j] = d * (float)sc;
            ms[j] = dmin * (float)mn;
        }
        const uint8_t* qs = blk + 16;
        const float* xb = x + (size_t)b * ORC_QK_K;
        for (int c = 0; c < 4; c++) {
            const uint8_t* q = qs + 32 * c;
            const float* xi = xb + 64 * c;
            /* low nibbles: groups of 8 alternate acc0/acc1 (:108-111) */
            for (int g = 0; g < 4; g++) {
                float* acc = (g & 1) ? a1 : a0;
                for (int k = 0; k < 8; k++) {
                    const float w = fmaf(ds[2 * c], (float)(q[8 * g + k] & 0x0f), -ms[2 * c]);
                    acc[k] = fmaf(w, xi[8 * g + k], acc[k]);
                }
            }
            /* high nibbles (:114-117) */
            for (int g = 0; g < 4; g++) {
                float* acc = (g & 1) ? a1 : a0;
                for (int k = 0; k < 8; k++) {
                    const float w = fmaf(ds[2 * c + 1], (float)(q[8 * g + k] >> 4), -ms[2 * c + 1]);
                    acc[k] = fmaf(w, xi[32 + 8 * g + k], acc[k]);
                }
            }
        }
    }
    float v[8];
    for (int k = 0; k < 8; k++) v[k] = a0[k] + a1[k];
    return hsum8(v);
}

void orc_gemv_q4k_f32(float* y, const uint8_t* W, const float* x, int o_start, int o_end,
                      int in_dim, size_t row_bytes) {
    for (int o = o_start; o < o_end; o++) y[o] = q4k_f32_row(W + (size_t)o * row_bytes, x, in_dim);
}

/* One 32-element Q6_K stream against x (accum_stream_q6_, gemv_q6k_avx2.cpp:66-88):
 * elements 0-7 -> acc0, 8-15 -> acc1 (scale0); 16-23 -> acc0, 24-31 -> acc1 (scale1);
 * weight = fmsub(s, q_raw, s*32). */
static void q6_stream_f32(const uint8_t* q, const float* x, float s0, float s1, float* a0,
                          float* a1) {
    const float b0 = s0 * 32.f, b1 = s1 * 32.f;
    for (int g = 0; g < 4; g++) {
        float* acc = (g & 1) ? a1 : a0;
        const float s = g < 2 ? s0 : s1;
        const float bb = g < 2 ? b0 : b1;
        for (int k = 0; k < 8; k++) {
            const float w = fmaf(s, (float)q[8 * g + k], -bb);
            acc[k] = fmaf(w, x[8 * g + k], acc[k]);
        }
    }
}

/* One row of gemv_q6k_avx2_range (gemv_q6k_avx2.cpp:91-149; 4-row tile
 * :154-233 has the same per-row sequence). */
static float q6k_f32_row(const uint8_t* row, const float* x, int in_dim) {
    float a0[8] = {0}, a1[8] = {0};
    const int nb = in_dim / ORC_QK_K;
    for (int b = 0; b < nb; b++) {
        const uint8_t* blk = row + (size_t)b * ORC_Q6K_BYTES;
        const float d = orc_fp16_to_fp32(rd16(blk + 208));
        const int8_t* scb = (const int8_t*)(blk + 192);
        for (int n = 0; n < 2; n++) {
            const uint8_t* ql = blk + 64 * n;
            const uint8_t* qh = blk + 128 + 32 * n;
            const int8_t* sc = scb + 8 * n;
            const float* xp = x + (size_t)b * ORC_QK_K + 128 * n;
            uint8_t q1[32], q2[32], q3[32], q4[32];
            for (int l = 0; l < 32; l++) {
                q1[l] = (uint8_t)((ql[l] & 0x0f) | ((qh[l] & 3) << 4));
                q2[l] = (uint8_t)((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4));
                q3[l] = (uint8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4));
                q4[l] = (uint8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4));
            }
            q6_stream_f32(q1, xp + 0, d * (float)sc[0], d * (float)sc[1], a0, a1);
            q6_stream_f32(q2, xp + 32, d * (float)sc[2], d * (float)sc[3], a0, a1);
            q6_stream_f32(q3, xp + 64, d * (float)sc[4], d * (float)sc[5], a0, a1);
            q6_stream_f32(q4, xp + 96, d * (float)sc[6], d * (float)sc[7], a0, a1);
        }
    }
    float v[8];
    for (int k = 0; k < 8; k++) v[k] = a0[k] + a1[k];
    return hsum8(v);
}

void orc_gemv_q6k_f32(float* y, const uint8_t* W, const float* x, int o_start, int o_end,
                      int in_dim, size_t row_bytes) {
    for (int o = o_start; o < o_end; o++) y[o] = q6k_f32_row(W + (size_t)o * row_bytes, x, in_dim);
}

/* ------------------------------------------------------------------------ */
/* Q8_0 activation path                                                     */
/* ------------------------------------------------------------------------ */

/* quantize_q8_avx2, quant_q8_avx2.cpp:33-84: d = amax/127, id = 127/amax,
 * q = cvtps_epi32(x*id) (round-to-nearest-even), saturating packs to int8. */
void orc_quantize_q8_0(orc_block_q8_0* y, const float* x, int k) {
    const int nb = k / 32;
    for (int i = 0; i < nb; i++) {
        const float* src = x + (size_t)i * 32;
        float amax = 0.f;
        for (int j = 0; j < 32; j++) {
            const float a = fabsf(src[j]);
            amax = a > amax ? a : amax;
        }
        const float d = amax / 127.f;
        const float id = (amax > 0.f) ? 127.f / amax : 0.f;
        y[i].d = d;
        for (int j = 0; j < 32; j++) {
            /* _mm256_cvtps_epi32 returns INT_MIN (the integer indefinite) for
             * a product outside the int32 range, inf or NaN: 0 < amax < 127/FLT_MAX
             * makes id = +inf and every product +-inf or NaN, so every value of
             * such a block packs to -128 */
            const float pr = src[j] * id;
            int q;
            if (!(fabsf(pr) < 2147483648.f)) {
                q = -128;
            } else {
                const float r = rintf(pr);
                q = (r > 127.f) ? 127 : (r < -128.f) ? -128 : (int)r;
            }
            y[i].qs[j] = (int8_t)q;
        }
    }
}

/* One row of the Q4_K x Q8_0 GEMV.  gemv_q4k_r8_avxvnni_range
 * (gemv_q4k_r8_avxvnni.cpp:76-183), gemv_q4k_r8_avx2_range
 * (gemv_q4k_r8_avx2.cpp:142-254) and the 4-row/1-row kernels of
 * gemv_q4k_q8_{avx2,avxvnni}.cpp all perform this per-row sequence:
 *   lane k of dot   = sum of nib*q8 over bytes 4k..4k+3   (dpbusd / maddubs+madd)
 *   lane k of sum   = q8[2k]+q8[2k+1]+q8[2k+16]+q8[2k+17] (q8_sum_f32_r8_)
 *   acc = fmadd(ds*dx, dot, acc); acc = fnmadd(ms*dx, sum, acc)   (low nibbles, g0)
 *   same for the high nibbles with g1; one hsum at the end of the row. */
static float q4k_q8_row(const uint8_t* row, const orc_block_q8_0* xq8, int in_dim) {
    float acc[8] = {0};
    const int nb = in_dim / ORC_QK_K;
    for (int b = 0; b < nb; b++) {
        const uint8_t* blk = row + (size_t)b * ORC_Q4K_BYTES;
        const float fd = orc_fp16_to_fp32(rd16(blk));
        const float fdm = orc_fp16_to_fp32(rd16(blk + 2));
        float ds[8], ms[8];
        for (int j = 0; j < 8; j++) {
            uint8_t sc, mn;
            orc_get_scale_min_k4(j, blk + 4, &sc, &mn);
            ds[j] = (float)sc * fd;
            ms[j] = (float)mn * fdm;
        }
        const orc_block_q8_0* xb = xq8 + (size_t)b * 8;
        for (int c = 0; c < 4; c++) {
            const int g0 = 2 * c, g1 = 2 * c + 1;
            const uint8_t* q = blk + 16 + 32 * c;
            const int8_t* x0 = xb[g0].qs;
            const int8_t* x1 = xb[g1].qs;
            const float d0 = xb[g0].d, d1 = xb[g1].d;
            const float s0 = ds[g0] * d0, m0 = ms[g0] * d0;
            const float s1 = ds[g1] * d1, m1 = ms[g1] * d1;
            for (int k = 0; k < 8; k++) {
                int dot_lo = 0, dot_hi = 0;
                for (int i = 4 * k; i < 4 * k + 4; i++) {
                    dot_lo += (q[i] & 0x0f) * x0[i];
                    dot_hi += (q[i] >> 4) * x1[i];
                }
                const int sum0 = x0[2 * k] + x0[2 * k + 1] + x0[2 * k + 16] + x0[2 * k + 17];
                const int sum1 = x1[2 * k] + x1[2 * k + 1] + x1[2 * k + 16] + x1[2 * k + 17];
                acc[k] = fmaf(s0, (float)dot_lo, acc[k]);
                acc[k] = fmaf(-m0, (float)sum0, acc[k]);
                acc[k] = fmaf(s1, (float)dot_hi, acc[k]);
                acc[k] = fmaf(-m1, (float)sum1, acc[k]);
            }
        }
    }
    return hsum8(acc);
}

void orc_gemv_q4k_q8(float* y, const uint8_t* W, const orc_block_q8_0* xq8, int o_start,
                     int o_end, int in_dim, size_t row_bytes) {
    for (int o = o_start; o < o_end; o++) y[o] = q4k_q8_row(W + (size_t)o * row_bytes, xq8, in_dim);
}

/* One row of gemv_q6k_q8_avx2_range (gemv_q6k_q8_avx2.cpp:104-205).
 *   lane k of dot = sum of q6*q8 over bytes 4k..4k+3 (maddubs+madd per 128-bit half)
 *   sum lanes from hadd_epi32 (q8_sum_hadd_f32_q6_, :50-56):
 *     0:q[0..3] 1:q[4..7] 2:q[16..19] 3:q[20..23] 4:q[8..11] 5:q[12..15] 6:q[24..27] 7:q[28..31]
 *   scale_dot lanes 0-3 sc0, 4-7 sc1; scale_corr lanes {0,1,4,5} sc0, {2,3,6,7} sc1
 *   acc = fmadd(scale_dot*dx, dot, acc); acc = fnmadd((scale_corr*dx)*32, sum, acc). */
static const int q6_sum_start[8] = {0, 4, 16, 20, 8, 12, 24, 28};
static const int q6_corr_hi[8] = {0, 0, 1, 1, 0, 0, 1, 1};

static float q6k_q8_row(const uint8_t* row, const orc_block_q8_0* xq8, int in_dim) {
    float acc[8] = {0};
    const int nb = in_dim / ORC_QK_K;
    for (int b = 0; b < nb; b++) {
        const uint8_t* blk = row + (size_t)b * ORC_Q6K_BYTES;
        const float fd = orc_fp16_to_fp32(rd16(blk + 208));
        const int8_t* scp = (const int8_t*)(blk + 192);
        const orc_block_q8_0* xb = xq8 + (size_t)b * 8;
        for (int half = 0; half < 2; half++) {
            const uint8_t* ql = blk + 64 * half;
            const uint8_t* qh = blk + 128 + 32 * half;
            const int8_t* sch = scp + 8 * half;
            for (int s = 0; s < 4; s++) {
                const uint8_t* qls = ql + (s & 1) * 32;
                uint8_t q6[32];
                for (int l = 0; l < 32; l++) {
                    const int lo4 = (s < 2) ? (qls[l] & 0x0f) : (qls[l] >> 4);
                    const int hi2 = (qh[l] >> (2 * s)) & 3;
                    q6[l] = (uint8_t)((lo4 | (hi2 << 4)) & 0x3f);
                }
                const orc_block_q8_0* xq = &xb[half * 4 + s];
                const float q8d = xq->d;
                const float sc0 = fd * (float)sch[2 * s];
                const float sc1 = fd * (float)sch[2 * s + 1];
                for (int k = 0; k < 8; k++) {
                    int dot = 0;
                    for (int i = 4 * k; i < 4 * k + 4; i++) dot += q6[i] * xq->qs[i];
                    const int st = q6_sum_start[k];
                    const int sum = xq->qs[st] + xq->qs[st + 1] + xq->qs[st + 2] + xq->qs[st + 3];
                    const float sdot = (k < 4 ? sc0 : sc1) * q8d;
                    const float scor = ((q6_corr_hi[k] ? sc1 : sc0) * q8d) * 32.f;
                    acc[k] = fmaf(sdot, (float)dot, acc[k]);
                    acc[k] = fmaf(-scor, (float)sum, acc[k]);
                }
            }
        }
    }
    return hsum8(acc);
}

void orc_gemv_q6k_q8(float* y, const uint8_t* W, const orc_block_q8_0* xq8, int o_start,
                     int o_end, int in_dim, size_t row_bytes) {
    for (int o = o_start; o < o_end; o++) y[o] = q6k_q8_row(W + (size_t)o * row_bytes, xq8, in_dim);
}

/* repack_q4k_8rows, gemv_q4k_r8_avx2.cpp:102-136: per (8-row group, block):
 * d[8] @0, dmin[8] @16, scales[8x12] @32, qs chunk c row r @128+256c+32r. */
void orc_repack_q4k_r8(uint8_t* dst, const uint8_t* src, int nrows, int ncols) {
    const int nb = ncols / ORC_QK_K;
    const size_t row_bytes = (size_t)nb * ORC_Q4K_BYTES;
    for (int g = 0; g < nrows / 8; g++) {
        for (int b = 0; b < nb; b++) {
            uint8_t* out = dst + ((size_t)g * nb + b) * 1152;
            for (int r = 0; r < 8; r++) {
                const uint8_t* blk = src + (size_t)(g * 8 + r) * row_bytes + (size_t)b * ORC_Q4K_BYTES;
                memcpy(out + 2 * r, blk, 2);
                memcpy(out + 16 + 2 * r, blk + 2, 2);
                memcpy(out + 32 + 12 * r, blk + 4, 12);
                for (int c = 0; c < 4; c++) memcpy(out + 128 + 256 * c + 32 * r, blk + 16 + 32 * c, 32);
            }
        }
    }
}

/* gemm_q4k_q8_avx2_range, gemv_q4k_q8_avx2.cpp:257-346: 4-row x 8-token tiles
 * with scalar fp32 accumulation of
 *   ds0*dq0*dot0 - ms0*(dq0*sum0) + ds1*dq1*dot1 - ms1*(dq1*sum1)
 * (integer dot and sum exact); rows outside 4-row tiles use the GEMV row.
 * Y is token-major: Y[t*M + m].  GCC 11 (-O3 -mfma) contracts the scalar
 * expression into three FMAs followed by the add into acc; the restatement
 * uses the same contraction (probed on the expression, checked against
 * oracle/_ref in tests). */
void orc_gemm_q4k_q8(float* Y, const uint8_t* W, const orc_block_q8_0* XQ8, int M, int T,
                     int K, size_t row_bytes, int o_start, int o_end) {
    const int nb = K / ORC_QK_K;
    const int bpt = K / 32;
    int o = o_start;
    for (; o + 4 <= o_end; o += 4) {
        for (int t0 = 0; t0 < T; t0 += 8) {
            const int nt = (T - t0) < 8 ? (T - t0) : 8;
            float acc[4][8];
            memset(acc, 0, sizeof(acc));
            for (int b = 0; b < nb; b++) {
                float ds[4][8], ms[4][8];
                const uint8_t* blk[4];
                for (int r = 0; r < 4; r++) {
                    blk[r] = W + (size_t)(o + r) * row_bytes + (size_t)b * ORC_Q4K_BYTES;
                    const float fd = orc_fp16_to_fp32(rd16(blk[r]));
                    const float fdm = orc_fp16_to_fp32(rd16(blk[r] + 2));
                    for (int j = 0; j < 8; j++) {
                        uint8_t sc, mn;
                        orc_get_scale_min_k4(j, blk[r] + 4, &sc, &mn);
                        ds[r][j] = fd * (float)sc;
                        ms[r][j] = fdm * (float)mn;
                    }
                }
                for (int c = 0; c < 4; c++) {
                    const int g0 = 2 * c, g1 = 2 * c + 1;
                    for (int ti = 0; ti < nt; ti++) {
                        const orc_block_q8_0* xb = XQ8 + (size_t)(t0 + ti) * bpt + (size_t)b * 8;
                        int sum0 = 0, sum1 = 0;
                        for (int i = 0; i < 32; i++) {
                            sum0 += xb[g0].qs[i];
                            sum1 += xb[g1].qs[i];
                        }
                        const float dq0 = xb[g0].d, dq1 = xb[g1].d;
                        const float contrib0 = dq0 * (float)sum0;
                        const float contrib1 = dq1 * (float)sum1;
                        for (int r = 0; r < 4; r++) {
                            const uint8_t* q = blk[r] + 16 + 32 * c;
                            int dot0 = 0, dot1 = 0;
                            for (int i = 0; i < 32; i++) {
                                dot0 += (q[i] & 0x0f) * xb[g0].qs[i];
                                dot1 += (q[i] >> 4) * xb[g1].qs[i];
                            }
                            /* contraction as GCC 11 -O3 -mfma emits for this expression */
                            const float u = fmaf(ds[r][g0] * dq0, (float)dot0, -(ms[r][g0] * contrib0));
                            const float v = fmaf(ds[r][g1] * dq1, (float)dot1, u);
                            const float w = fmaf(-ms[r][g1], contrib1, v);
                            acc[r][ti] = acc[r][ti] + w;
                        }
                    }
                }
            }
            for (int r = 0; r < 4; r++)
                for (int ti = 0; ti < nt; ti++) Y[(size_t)(t0 + ti) * M + o + r] = acc[r][ti];
        }
    }
    for (; o < o_end; o++)
        for (int t = 0; t < T; t++)
            Y[(size_t)t * M + o] = q4k_q8_row(W + (size_t)o * row_bytes, XQ8 + (size_t)t * bpt, K);
}

/* ------------------------------------------------------------------------ */
/* decode-step operations                                                   */
/* ------------------------------------------------------------------------ */

/* rms_norm_out, llama_model.cpp:396-419 (and rms_norm_avx2 :371-393 in place):
 * 8-lane fmadd of x^2, scalar sum of the 8 lanes, s = 1/sqrt(ss/n + eps),
 * y = w*(x*s) for the vector part. */
void orc_rmsnorm(float* dst, const float* src, const float* w, int n, float eps) {
    float acc[8] = {0};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int k = 0; k < 8; k++) acc[k] = fmaf(src[i + k], src[i + k], acc[k]);
    float ss = 0.f;
    for (int k = 0; k < 8; k++) ss += acc[k];
    for (; i < n; i++) ss += src[i] * src[i];
    ss = 1.f / sqrtf(ss / (float)n + eps);
    i = 0;
    for (; i + 8 <= n; i += 8)
        for (int k = 0; k < 8; k++) dst[i + k] = w[i + k] * (src[i + k] * ss);
    for (; i < n; i++) dst[i] = w[i] * src[i] * ss;
}

void orc_rmsnorm_heads(float* x, const float* w, int n_heads, int head_dim, float eps) {
    if (!w) return;
    for (int h = 0; h < n_heads; h++)
        orc_rmsnorm(x + (size_t)h * head_dim, x + (size_t)h * head_dim, w, head_dim, eps);
}

/* RopeCache::build, llama_model.cpp:1031-1043 (glibc powf/cosf/sinf). */
void orc_rope_table(float* cos_t, float* sin_t, int hd, float theta, int max_pos) {
    const int half = hd / 2;
    for (int p = 0; p < max_pos; p++) {
        for (int i = 0; i < half; i++) {
            const float freq = 1.f / powf(theta, (float)(2 * i) / (float)hd);
            const float angle = (float)p * freq;
            cos_t[(size_t)p * half + i] = cosf(angle);
            sin_t[(size_t)p * half + i] = sinf(angle);
        }
    }
}

/* apply_rope / rope_and_store_k, llama_model.cpp:1046-1080: rotate-half pairs
 * (i, i+hd/2).  GCC 11 -O3 -mfma contracts the two expressions as
 *   x0*c - x1*s -> fma(x0, c, -(x1*s)),  x0*s + x1*c -> fma(x0, s, x1*c).
 * dst may alias src. */
void orc_rope(float* dst, const float* src, int pos, int n_heads, int hd, const float* cos_t,
              const float* sin_t) {
    const int half = hd / 2;
    const float* cr = cos_t + (size_t)pos * half;
    const float* sr = sin_t + (size_t)pos * half;
    for (int h = 0; h < n_heads; h++) {
        const float* s = src + (size_t)h * hd;
        float* d = dst + (size_t)h * hd;
        for (int i = 0; i < half; i++) {
            const float x0 = s[i], x1 = s[i + half];
            const float a = fmaf(x0, cr[i], -(x1 * sr[i]));
            const float b = fmaf(x0, sr[i], x1 * cr[i]);
            d[i] = a;
            d[i + half] = b;
        }
    }
}

/* avx2_dot_f32, llama_model.cpp:1169-1190: two 8-lane accumulators over
 * 16-element steps, one 8-element step, lane add, hsum, scalar tail. */
float orc_dot_f32(const float* a, const float* b, int n) {
    float a0[8] = {0}, a1[8] = {0};
    int i = 0;
    for (; i + 16 <= n; i += 16)
        for (int k = 0; k < 8; k++) {
            a0[k] = fmaf(a[i + k], b[i + k], a0[k]);
            a1[k] = fmaf(a[i + 8 + k], b[i + 8 + k], a1[k]);
        }
    for (; i + 8 <= n; i += 8)
        for (int k = 0; k < 8; k++) a0[k] = fmaf(a[i + k], b[i + k], a0[k]);
    float v[8];
    for (int k = 0; k < 8; k++) v[k] = a0[k] + a1[k];
    float s = hsum8(v);
    for (; i < n; i++) s += a[i] * b[i];
    return s;
}

/* softmax, llama_model.cpp:445-451 (glibc expf, sequential sum, divide). */
void orc_softmax(float* x, int n) {
    float mx = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float sum = 0.f;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    for (int i = 0; i < n; i++) x[i] /= sum;
}

/* Single-token GQA attention, llama_model.cpp:1255-1272: per head
 * score[t] = dot(q_h, k_t)*(1/sqrt(hd)), softmax, out_h += p[t]*v_t (8-lane
 * fmadd saxpy, :1193-1203).  kcache/vcache rows hold n_kv_heads*hd floats. */
void orc_attention(float* out, const float* q, const float* kcache, const float* vcache,
                   int seq, int n_heads, int n_kv_heads, int hd, float* scores) {
    const float scale = 1.f / sqrtf((float)hd);
    const int group = n_heads / n_kv_heads;
    const size_t kv_embd = (size_t)n_kv_heads * hd;
    memset(out, 0, sizeof(float) * (size_t)n_heads * hd);
    for (int h = 0; h < n_heads; h++) {
        const int kvh = h / group;
        const float* qh = q + (size_t)h * hd;
        for (int t = 0; t < seq; t++)
            scores[t] = orc_dot_f32(qh, kcache + (size_t)t * kv_embd + (size_t)kvh * hd, hd) * scale;
        orc_softmax(scores, seq);
        float* oh = out + (size_t)h * hd;
        for (int t = 0; t < seq; t++) {
            const float* vt = vcache + (size_t)t * kv_embd + (size_t)kvh * hd;
            int i = 0;
            for (; i + 8 <= hd; i += 8)
                for (int k = 0; k < 8; k++) oh[i + k] = fmaf(scores[t], vt[i + k], oh[i + k]);
            for (; i < hd; i++) oh[i] += scores[t] * vt[i];
        }
    }
}

/* exp_avx2_, llama_model.cpp:319-344: the Cephes single-precision expf method
 * (Moshier, Cephes Math Library): clamp to +-88.376, n = floor(x*log2e + 1/2),
 * two-constant Cody-Waite reduction by ln2, degree-5 polynomial, scale by 2^n. */
float orc_exp_cephes(float x) {
    float xx = x < 88.3762626648f ? x : 88.3762626648f;
    xx = -88.3762626648f > xx ? -88.3762626648f : xx;
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
    const int32_t n = ((int32_t)fx + 127) << 23;
    float two_n;
    memcpy(&two_n, &n, 4);
    return p * two_n;
}

/* swiglu_avx2, llama_model.cpp:348-368: e = exp(-|g|), sigmoid = 1/(1+e)
 * for g >= 0 and e/(1+e) for g < 0; gate = (g*sigmoid)*up.  The scalar tail
 * (:367, x/(1+exp(-x))*up) only runs when n % 8 != 0. */
void orc_swiglu(float* gate, const float* up, int n) {
    int i = 0;
    for (; i + 8 <= n; i += 8) {
        for (int k = 0; k < 8; k++) {
            const float g = gate[i + k];
            const float e = orc_exp_cephes(-fabsf(g));
            const float denom = 1.f + e;
            const float sig = (g < 0.f) ? e / denom : 1.f / denom;
            gate[i + k] = (g * sig) * up[i + k];
        }
    }
    for (; i < n; i++) {
        const float g = gate[i];
        gate[i] = g / (1.f + expf(-g)) * up[i];
    }
}

/* Greedy sample: std::max_element (first index of the maximum),
 * llama_model.cpp:1470-1471. */
int orc_argmax(const float* x, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (x[best] < x[i]) best = i;
    return best;
}

float orc_top2_margin(const float* x, int n) {
    const int b = orc_argmax(x, n);
    float second = -INFINITY;
    for (int i = 0; i < n; i++)
        if (i != b && x[i] > second) second = x[i];
    return x[b] - second;
}

/* ------------------------------------------------------------------------ */
/* other weight types of the decode path                                    */
/* ------------------------------------------------------------------------ */

/* q8_0_weight_dot_q8_row (llama_model.cpp:171-211): per 34-byte block the
 * scale f16(d_w) * d_x times the exact int32 dot, summed in block order. */
void orc_gemv_q8_0w_q8(float* y, const uint8_t* W, const orc_block_q8_0* xq8, int o0, int o1,
                       int in, size_t rb) {
    const int nb = in / 32;
    for (int o = o0; o < o1; o++) {
        const uint8_t* row = W + (size_t)o * rb;
        float acc = 0.f;
        for (int b = 0; b < nb; b++) {
            const float scale = orc_fp16_to_fp32(rd16(row + (size_t)b * 34)) * xq8[b].d;
            const int8_t* q = (const int8_t*)(row + (size_t)b * 34 + 2);
            int isum = 0;
            for (int i = 0; i < 32; i++) isum += (int)q[i] * (int)xq8[b].qs[i];
            acc += scale * (float)isum;
        }
        y[o] = acc;
    }
}

/* q8_0_weight_dot_row (:154-169): acc += d * q * x element by element. */
void orc_gemv_q8_0w_f32(float* y, const uint8_t* W, const float* x, int o0, int o1, int in,
                        size_t rb) {
    const int nb = (in + 31) / 32;
    for (int o = o0; o < o1; o++) {
        const uint8_t* row = W + (size_t)o * rb;
        float acc = 0.f;
        for (int b = 0; b < nb; b++) {
            const float d = orc_fp16_to_fp32(rd16(row + (size_t)b * 34));
            const int8_t* q = (const int8_t*)(row + (size_t)b * 34 + 2);
            const int lim = in - b * 32 < 32 ? in - b * 32 : 32;
            for (int i = 0; i < lim; i++) acc += d * (float)q[i] * x[b * 32 + i];
        }
        y[o] = acc;
    }
}

/* Q5_0 element i of a block: low nibble of qs[i] (i < 16) or high nibble of
 * qs[i - 16], bit i of qh as bit 4; w = d * (q - 16) (q5_0_dot_row :245-267). */
static float q5_0_w(const uint8_t* blk, int i) {
    const float d = orc_fp16_to_fp32(rd16(blk));
    const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                        ((uint32_t)blk[5] << 24);
    const uint8_t* qs = blk + 6;
    const uint32_t nib = i < 16 ? (uint32_t)(qs[i] & 0x0f) : (uint32_t)(qs[i - 16] >> 4);
    const uint32_t hi = (qh >> i) & 1u;
    return d * ((float)(nib | (hi << 4)) - 16.f);
}

void orc_gemv_q5_0_f32(float* y, const uint8_t* W, const float* x, int o0, int o1, int in,
                       size_t rb) {
    const int nb = (in + 31) / 32;
    for (int o = o0; o < o1; o++) {
        const uint8_t* row = W + (size_t)o * rb;
        float acc = 0.f;
        for (int b = 0; b < nb; b++) {
            const int lim = in - b * 32 < 32 ? in - b * 32 : 32;
            for (int i = 0; i < lim; i++) acc += q5_0_w(row + (size_t)b * 22, i) * x[b * 32 + i];
        }
        y[o] = acc;
    }
}

/* gemv_f16_avx2_range (gemv_f16_avx2.cpp:98-153) with an __m256 restated as
 * float[8]: 4-row tiles (when no bias) with two 8-lane FMA accumulators per
 * row over 16-element steps, then one over an 8-element step, lane-wise add,
 * hsum8, scalar tail; remaining rows one at a time the same way (+ bias). */
static float f16_hsum8(const float* v) {
    float lo[4];
    for (int i = 0; i < 4; i++) lo[i] = v[i] + v[i + 4];
    const float h0 = lo[0] + lo[1], h1 = lo[2] + lo[3];
    return h0 + h1;
}

static float f16_dot_row(const uint16_t* w, const float* x, int in) {
    float a[8] = {0}, b[8] = {0};
    int k = 0;
    for (; k + 16 <= in; k += 16)
        for (int l = 0; l < 8; l++) {
            a[l] = fmaf(orc_fp16_to_fp32(w[k + l]), x[k + l], a[l]);
            b[l] = fmaf(orc_fp16_to_fp32(w[k + 8 + l]), x[k + 8 + l], b[l]);
        }
    for (; k + 8 <= in; k += 8)
        for (int l = 0; l < 8; l++) a[l] = fmaf(orc_fp16_to_fp32(w[k + l]), x[k + l], a[l]);
    for (int l = 0; l < 8; l++) a[l] += b[l];
    float sum = f16_hsum8(a);
    for (; k < in; k++) sum = fmaf(orc_fp16_to_fp32(w[k]), x[k], sum);
    return sum;
}

void orc_gemv_f16_f32(float* y, const uint16_t* W, const float* x, const float* bias, int o0,
                      int o1, int in) {
    for (int o = o0; o < o1; o++) {
        const float s = f16_dot_row(W + (size_t)o * in, x, in);
        y[o] = bias ? s + bias[o] : s;
    }
}

/* emb_lookup rows of the other types (llama_model.cpp:882-898): exact. */
void orc_dequant_row(float* out, int qtype, const uint8_t* row, int cols) {
    for (int i = 0; i < cols; i++) {
        if (qtype == 1) {
            out[i] = orc_fp16_to_fp32(rd16(row + 2 * i));
        } else if (qtype == 8) {
            const uint8_t* blk = row + (size_t)(i / 32) * 34;
            out[i] = orc_fp16_to_fp32(rd16(blk)) * (float)(int8_t)blk[2 + i % 32];
        } else {
            out[i] = q5_0_w(row + (size_t)(i / 32) * 22, i % 32);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* sampling (llama_generate_cpu_impl)                                        */
/* ------------------------------------------------------------------------ */

/* apply_rep_penalty (llama_model.cpp:1595-1605): the last min(last_n, n_hist)
 * history ids in order, each occurrence dividing a positive logit by the
 * penalty or multiplying a non-positive one. */
void orc_rep_penalty(float* logits, int n_vocab, const int32_t* hist, int n_hist, int last_n,
                     float penalty) {
    if (penalty == 1.0f) return;
    const int win = last_n < n_hist ? last_n : n_hist;
    for (int i = n_hist - win; i < n_hist; i++) {
        const int32_t id = hist[i];
        if (id < 0 || id >= n_vocab) continue;
        logits[id] = logits[id] > 0.f ? logits[id] / penalty : logits[id] * penalty;
    }
}

typedef struct {
    float v;
    int32_t i;
} orc_scored;

/* value descending; equal values by index ascending (the reference's
 * partial_sort leaves their order unspecified) */
static int scored_cmp(const void* pa, const void* pb) {
    const orc_scored* a = (const orc_scored*)pa;
    const orc_scored* b = (const orc_scored*)pb;
    if (a->v > b->v) return -1;
    if (a->v < b->v) return 1;
    return (a->i > b->i) - (a->i < b->i);
}

static float fminabs(float m, float d) {
    d = fabsf(d);
    return d < m ? d : m;
}

/* sample() (llama_model.cpp:1466-1498) with the uniform draw r.  *margin is
 * the distance of the decision from flipping: |r - cum| at the chosen entry
 * and the one before it, and |cum - top_p| at the nucleus cut (FLT_MAX for
 * greedy). */
int orc_sample(const float* logits, int n_vocab, int top_k, float top_p, float temperature,
               float r, float* margin) {
    if (margin) *margin = FLT_MAX;
    if (temperature <= 0.f) return orc_argmax(logits, n_vocab);
    int k = (top_k > 0 && top_k < n_vocab) ? top_k : n_vocab;
    orc_scored* sc = (orc_scored*)malloc(sizeof(orc_scored) * (size_t)n_vocab);
    float* probs = (float*)malloc(sizeof(float) * (size_t)n_vocab);
    for (int i = 0; i < n_vocab; i++) {
        sc[i].v = logits[i] / temperature;
        sc[i].i = i;
    }
    qsort(sc, (size_t)n_vocab, sizeof(orc_scored), scored_cmp);
    const float mx = sc[0].v;
    float sum = 0.f, m = FLT_MAX;
    for (int i = 0; i < k; i++) {
        probs[i] = expf(sc[i].v - mx);
        sum += probs[i];
    }
    for (int i = 0; i < k; i++) probs[i] /= sum;
    if (top_p < 1.0f) {
        float cum = 0.f;
        int cut = k;
        for (int i = 0; i < k; i++) {
            cum += probs[i];
            m = fminabs(m, cum - top_p);
            if (cum >= top_p) {
                cut = i + 1;
                break;
            }
        }
        sum = 0.f;
        for (int i = 0; i < cut; i++) sum += probs[i];
        for (int i = 0; i < cut; i++) probs[i] /= sum;
        k = cut;
    }
    float cum = 0.f;
    int chosen = sc[k - 1].i;
    for (int i = 0; i < k; i++) {
        cum += probs[i];
        m = fminabs(m, r - cum);
        if (r < cum) {
            chosen = sc[i].i;
            break;
        }
    }
    free(sc);
    free(probs);
    if (margin) *margin = m;
    return chosen;
}

/* ------------------------------------------------------------------------ */
/* decoder (llama_forward_token / llama_forward_batch)                       */
/* ------------------------------------------------------------------------ */

struct orc_state {
    int n_ctx, kv_embd, hd;
    float *x, *xb, *q, *k, *v, *attn, *attn_out, *gate, *up, *ffn, *logits;
    orc_block_q8_0* xq8;
    float *kv_k, *kv_v; /* [n_layer][n_ctx][kv_embd], LlamaState :1102-1106 */
    float *rope_cos, *rope_sin;
};

orc_state* orc_state_new(const orc_model* m) {
    orc_state* s = (orc_state*)calloc(1, sizeof(orc_state));
    const int E = m->n_embd, FD = m->ffn_dim;
    s->n_ctx = m->n_ctx;
    s->hd = E / m->n_heads;
    s->kv_embd = m->n_kv_heads * s->hd;
    s->x = (float*)calloc((size_t)E, 4);
    s->xb = (float*)calloc((size_t)E, 4);
    s->q = (float*)calloc((size_t)E, 4);
    s->k = (float*)calloc((size_t)s->kv_embd, 4);
    s->v = (float*)calloc((size_t)s->kv_embd, 4);
    s->attn = (float*)calloc((size_t)m->n_ctx, 4);
    s->attn_out = (float*)calloc((size_t)E, 4);
    s->gate = (float*)calloc((size_t)FD, 4);
    s->up = (float*)calloc((size_t)FD, 4);
    s->ffn = (float*)calloc((size_t)E, 4);
    s->logits = (float*)calloc((size_t)m->n_vocab, 4);
    s->xq8 = (orc_block_q8_0*)calloc((size_t)((E > FD ? E : FD) / 32), sizeof(orc_block_q8_0));
    s->kv_k = (float*)calloc((size_t)m->n_layer * m->n_ctx * s->kv_embd, 4);
    s->kv_v = (float*)calloc((size_t)m->n_layer * m->n_ctx * s->kv_embd, 4);
    s->rope_cos = (float*)calloc((size_t)m->n_ctx * (s->hd / 2), 4);
    s->rope_sin = (float*)calloc((size_t)m->n_ctx * (s->hd / 2), 4);
    orc_rope_table(s->rope_cos, s->rope_sin, s->hd, m->rope_theta, m->n_ctx);
    return s;
}

void orc_state_free(orc_state* s) {
    if (!s) return;
    free(s->x); free(s->xb); free(s->q); free(s->k); free(s->v); free(s->attn);
    free(s->attn_out); free(s->gate); free(s->up); free(s->ffn); free(s->logits);
    free(s->xq8); free(s->kv_k); free(s->kv_v); free(s->rope_cos); free(s->rope_sin);
    free(s);
}

float* orc_state_logits(orc_state* s) { return s->logits; }
float* orc_state_x(orc_state* s) { return s->x; }
float* orc_state_kv_k(orc_state* s) { return s->kv_k; }
float* orc_state_kv_v(orc_state* s) { return s->kv_v; }
/* Intermediates of the last orc_forward_layer: q after bias and RoPE, the
 * attention output, and the SwiGLU output h (the down projection's input). */
float* orc_state_q(orc_state* s) { return s->q; }
float* orc_state_attn_out(orc_state* s) { return s->attn_out; }
float* orc_state_h(orc_state* s) { return s->gate; }

static size_t wt_row_bytes(const orc_wt* w, int in) {
    if (w->type == 8) return (size_t)((in + 31) / 32) * 34;  /* Q8_0 */
    if (w->type == 6) return (size_t)((in + 31) / 32) * 22;  /* Q5_0 */
    if (w->type == 1) return (size_t)in * 2;                 /* F16 */
    return (size_t)(in / ORC_QK_K) * (w->type == ORC_TYPE_Q6_K ? ORC_Q6K_BYTES : ORC_Q4K_BYTES);
}

/* gemv_wt, llama_model.cpp:670-731: fp32 activations. F16 -> the F16 GEMV
 * (:672-680), Q4_K / Q6_K -> the fp32-activation K-quant GEMVs (:681-700),
 * Q8_0 -> q8_0_weight_dot_row (:701-712), Q5_0 -> q5_0_dot_row (:713-724). */
static void gemv_wt(float* y, const orc_wt* w, const float* x, int out, int in) {
    const size_t rb = wt_row_bytes(w, in);
    if (w->type == 1)
        orc_gemv_f16_f32(y, (const uint16_t*)w->data, x, NULL, 0, out, in);
    else if (w->type == ORC_TYPE_Q4_K)
        orc_gemv_q4k_f32(y, w->data, x, 0, out, in, rb);
    else if (w->type == ORC_TYPE_Q6_K)
        orc_gemv_q6k_f32(y, w->data, x, 0, out, in, rb);
    else if (w->type == 8)
        orc_gemv_q8_0w_f32(y, w->data, x, 0, out, in, rb);
    else
        orc_gemv_q5_0_f32(y, w->data, x, 0, out, in, rb);
}

/* gemv_wt_q8, llama_model.cpp:767-831 (the decode step's GEMV; q8_fast and AVX2,
 * as the reference builds every layer, :986-1006): Q4_K and Q6_K -> the Q8_0
 * GEMVs, Q8_0 -> gemv_q8_0_weight_q8 (:825-828), everything else -> gemv_wt
 * with the fp32 activation xf32 (:830). */
static void gemv_wt_q8(float* y, const orc_wt* w, const orc_block_q8_0* xq8, const float* xf32,
                       int out, int in) {
    const size_t rb = wt_row_bytes(w, in);
    if (w->type == ORC_TYPE_Q6_K)
        orc_gemv_q6k_q8(y, w->data, xq8, 0, out, in, rb);
    else if (w->type == ORC_TYPE_Q4_K)
        orc_gemv_q4k_q8(y, w->data, xq8, 0, out, in, rb);
    else if (w->type == 8)
        orc_gemv_q8_0w_q8(y, w->data, xq8, 0, out, in, rb);
    else
        gemv_wt(y, w, xf32, out, in);
}

/* gemm_wt_q8, llama_model.cpp:837-879: Q4_K -> GEMM kernel; Q6_K -> per-token
 * Q8_0 GEMV; every other type (Q8_0 included: the batched path has no Q8_0
 * branch) -> gemv_wt per token with the fp32 rows XF32 (:876-879). */
static void gemm_wt_q8(float* Y, const orc_wt* w, const orc_block_q8_0* XQ8, const float* XF32,
                       int M, int T, int in) {
    const size_t rb = wt_row_bytes(w, in);
    if (w->type == ORC_TYPE_Q6_K) {
        for (int t = 0; t < T; t++)
            orc_gemv_q6k_q8(Y + (size_t)t * M, w->data, XQ8 + (size_t)t * (in / 32), 0, M, in, rb);
    } else if (w->type == ORC_TYPE_Q4_K) {
        orc_gemm_q4k_q8(Y, w->data, XQ8, M, T, in, rb, 0, M);
    } else {
        for (int t = 0; t < T; t++) gemv_wt(Y + (size_t)t * M, w, XF32 + (size_t)t * in, M, in);
    }
}

/* The head's gemv_wt_q8 (llama_model.cpp:1330-1332): the same dispatch. */
static void head_gemv(float* y, const orc_wt* w, const orc_block_q8_0* xq8, const float* x,
                      int out, int in) {
    gemv_wt_q8(y, w, xq8, x, out, in);
}

/* emb_lookup, llama_model.cpp:882-934. */
static void emb_lookup(float* out, const orc_wt* w, int row, int cols) {
    const int nb = cols / ORC_QK_K;
    const uint8_t* p = w->data + (size_t)row * wt_row_bytes(w, cols);
    if (w->type == 8 || w->type == 6 || w->type == 1)
        orc_dequant_row(out, w->type, p, cols);
    else if (w->type == ORC_TYPE_Q6_K)
        orc_dequant_q6k(out, p, nb);
    else
        orc_dequant_q4k(out, p, nb);
}

static void add_bias(float* y, const float* b, int n) {
    if (!b) return;
    for (int i = 0; i < n; i++) y[i] += b[i];
}

/* One decoder layer of llama_forward_token (llama_model.cpp:1222-1325) at
 * position pos; reads and updates s->x. */
void orc_forward_layer(const orc_model* m, orc_state* s, int l, int pos) {
    const int E = m->n_embd, H = m->n_heads, KVH = m->n_kv_heads, HD = s->hd, FD = m->ffn_dim;
    const orc_layer* lw = &m->layers[l];
    const size_t layer_off = (size_t)l * m->n_ctx * s->kv_embd;
    float* kc = s->kv_k + layer_off;
    float* vc = s->kv_v + layer_off;

    orc_rmsnorm(s->xb, s->x, lw->attn_norm, E, m->rms_eps);
    orc_quantize_q8_0(s->xq8, s->xb, E);
    gemv_wt_q8(s->q, &lw->wq, s->xq8, s->xb, H * HD, E);
    gemv_wt_q8(s->k, &lw->wk, s->xq8, s->xb, KVH * HD, E);
    gemv_wt_q8(s->v, &lw->wv, s->xq8, s->xb, KVH * HD, E);
    add_bias(s->q, lw->bq, H * HD);
    add_bias(s->k, lw->bk, KVH * HD);
    add_bias(s->v, lw->bv, KVH * HD);
    /* per-head q/k norms (:1236-1248): before RoPE, or after it (K normed in
     * the cache row, the same values the reference copies there) */
    float* krow = kc + (size_t)pos * s->kv_embd;
    if (m->qk_norm_order == ORC_QK_BEFORE_ROPE) {
        orc_rmsnorm_heads(s->q, lw->q_norm, H, HD, m->rms_eps);
        orc_rmsnorm_heads(s->k, lw->k_norm, KVH, HD, m->rms_eps);
    }
    orc_rope(s->q, s->q, pos, H, HD, s->rope_cos, s->rope_sin);
    orc_rope(krow, s->k, pos, KVH, HD, s->rope_cos, s->rope_sin);
    if (m->qk_norm_order == ORC_QK_AFTER_ROPE) {
        orc_rmsnorm_heads(s->q, lw->q_norm, H, HD, m->rms_eps);
        orc_rmsnorm_heads(krow, lw->k_norm, KVH, HD, m->rms_eps);
    }
    memcpy(vc + (size_t)pos * s->kv_embd, s->v, sizeof(float) * (size_t)s->kv_embd);

    orc_attention(s->attn_out, s->q, kc, vc, pos + 1, H, KVH, HD, s->attn);

    orc_quantize_q8_0(s->xq8, s->attn_out, E);
    gemv_wt_q8(s->xb, &lw->wo, s->xq8, s->attn_out, E, E);
    for (int i = 0; i < E; i++) s->x[i] += s->xb[i];

    orc_rmsnorm(s->xb, s->x, lw->ffn_norm, E, m->rms_eps);
    orc_quantize_q8_0(s->xq8, s->xb, E);
    gemv_wt_q8(s->gate, &lw->wgate, s->xq8, s->xb, FD, E);
    gemv_wt_q8(s->up, &lw->wup, s->xq8, s->xb, FD, E);
    orc_swiglu(s->gate, s->up, FD);
    orc_quantize_q8_0(s->xq8, s->gate, FD);
    gemv_wt_q8(s->ffn, &lw->wdown, s->xq8, s->gate, E, FD);
    for (int i = 0; i < E; i++) s->x[i] += s->ffn[i];
}

/* llama_forward_token, llama_model.cpp:1207-1333. */
void orc_forward_token(const orc_model* m, orc_state* s, int token, int pos) {
    const int E = m->n_embd;
    emb_lookup(s->x, &m->tok_embd, token, E);
    for (int l = 0; l < m->n_layer; l++) orc_forward_layer(m, s, l, pos);
    orc_rmsnorm(s->x, s->x, m->output_norm, E, m->rms_eps);
    orc_quantize_q8_0(s->xq8, s->x, E);
    head_gemv(s->logits, &m->output, s->xq8, s->x, m->n_vocab, E);
}

/* llama_forward_batch, llama_model.cpp:1339-1462: batched prefill with the
 * GEMM kernel for Q4_K weights; only the last token's logits are produced. */
void orc_forward_batch(const orc_model* m, orc_state* s, const int32_t* tokens, int T,
                       int pos_start) {
    const int E = m->n_embd, H = m->n_heads, KVH = m->n_kv_heads, HD = s->hd, FD = m->ffn_dim;
    const int kve = s->kv_embd;
    float* X = (float*)calloc((size_t)T * E, 4);
    float* XB = (float*)calloc((size_t)T * E, 4);
    float* Q = (float*)calloc((size_t)T * H * HD, 4);
    float* K = (float*)calloc((size_t)T * kve, 4);
    float* V = (float*)calloc((size_t)T * kve, 4);
    float* AO = (float*)calloc((size_t)T * E, 4);
    float* GATE = (float*)calloc((size_t)T * FD, 4);
    float* UP = (float*)calloc((size_t)T * FD, 4);
    float* FFN = (float*)calloc((size_t)T * E, 4);
    orc_block_q8_0* XQE = (orc_block_q8_0*)calloc((size_t)T * (E / 32), sizeof(orc_block_q8_0));
    orc_block_q8_0* XQF = (orc_block_q8_0*)calloc((size_t)T * (FD / 32), sizeof(orc_block_q8_0));

    for (int t = 0; t < T; t++) emb_lookup(X + (size_t)t * E, &m->tok_embd, tokens[t], E);
    for (int l = 0; l < m->n_layer; l++) {
        const orc_layer* lw = &m->layers[l];
        const size_t layer_off = (size_t)l * m->n_ctx * kve;
        float* kc = s->kv_k + layer_off;
        float* vc = s->kv_v + layer_off;
        for (int t = 0; t < T; t++) {
            orc_rmsnorm(XB + (size_t)t * E, X + (size_t)t * E, lw->attn_norm, E, m->rms_eps);
            orc_quantize_q8_0(XQE + (size_t)t * (E / 32), XB + (size_t)t * E, E);
        }
        gemm_wt_q8(Q, &lw->wq, XQE, XB, H * HD, T, E);
        gemm_wt_q8(K, &lw->wk, XQE, XB, KVH * HD, T, E);
        gemm_wt_q8(V, &lw->wv, XQE, XB, KVH * HD, T, E);
        for (int t = 0; t < T; t++) {
            add_bias(Q + (size_t)t * H * HD, lw->bq, H * HD);
            add_bias(K + (size_t)t * kve, lw->bk, kve);
            add_bias(V + (size_t)t * kve, lw->bv, kve);
            if (m->qk_norm_order == ORC_QK_BEFORE_ROPE) {  /* :1388-1391 */
                orc_rmsnorm_heads(Q + (size_t)t * H * HD, lw->q_norm, H, HD, m->rms_eps);
                orc_rmsnorm_heads(K + (size_t)t * kve, lw->k_norm, KVH, HD, m->rms_eps);
            }
        }
        for (int t = 0; t < T; t++) {
            const int pos = pos_start + t;
            float* qrow = Q + (size_t)t * H * HD;
            float* krow = kc + (size_t)pos * kve;
            orc_rope(qrow, qrow, pos, H, HD, s->rope_cos, s->rope_sin);
            orc_rope(krow, K + (size_t)t * kve, pos, KVH, HD, s->rope_cos, s->rope_sin);
            if (m->qk_norm_order == ORC_QK_AFTER_ROPE) {  /* :1397-1403 */
                orc_rmsnorm_heads(qrow, lw->q_norm, H, HD, m->rms_eps);
                orc_rmsnorm_heads(krow, lw->k_norm, KVH, HD, m->rms_eps);
            }
            memcpy(vc + (size_t)pos * kve, V + (size_t)t * kve, sizeof(float) * (size_t)kve);
        }
        for (int t = 0; t < T; t++)
            orc_attention(AO + (size_t)t * E, Q + (size_t)t * H * HD, kc, vc, pos_start + t + 1, H,
                          KVH, HD, s->attn);
        for (int t = 0; t < T; t++)
            orc_quantize_q8_0(XQE + (size_t)t * (E / 32), AO + (size_t)t * E, E);
        gemm_wt_q8(XB, &lw->wo, XQE, AO, E, T, E);
        for (size_t i = 0; i < (size_t)T * E; i++) X[i] += XB[i];
        for (int t = 0; t < T; t++) {
            orc_rmsnorm(XB + (size_t)t * E, X + (size_t)t * E, lw->ffn_norm, E, m->rms_eps);
            orc_quantize_q8_0(XQE + (size_t)t * (E / 32), XB + (size_t)t * E, E);
        }
        gemm_wt_q8(GATE, &lw->wgate, XQE, XB, FD, T, E);
        gemm_wt_q8(UP, &lw->wup, XQE, XB, FD, T, E);
        for (int t = 0; t < T; t++) {
            orc_swiglu(GATE + (size_t)t * FD, UP + (size_t)t * FD, FD);
            orc_quantize_q8_0(XQF + (size_t)t * (FD / 32), GATE + (size_t)t * FD, FD);
        }
        gemm_wt_q8(FFN, &lw->wdown, XQF, GATE, E, T, FD);
        for (size_t i = 0; i < (size_t)T * E; i++) X[i] += FFN[i];
    }
    float* xl = X + (size_t)(T - 1) * E;
    orc_rmsnorm(xl, xl, m->output_norm, E, m->rms_eps);
    orc_quantize_q8_0(XQE, xl, E);
    head_gemv(s->logits, &m->output, XQE, xl, m->n_vocab, E);
    memcpy(s->x, xl, sizeof(float) * (size_t)E);
    free(X); free(XB); free(Q); free(K); free(V); free(AO); free(GATE); free(UP); free(FFN);
    free(XQE); free(XQF);
}

/* Greedy generation loop of llama_generate_cpu_impl (llama_model.cpp:1561-1624)
 * with temperature 0 and no EOS: the prompt is used as given (the caller
 * includes BOS), prefill is batched when n_prompt > 1 (or token-by-token when
 * batched_prefill == 0), and n_gen tokens are emitted.  out_margins[i] is the
 * top-1 minus top-2 logit of the distribution token i was taken from. */
int orc_generate_greedy(const orc_model* m, const int32_t* prompt, int n_prompt, int n_gen,
                        int batched_prefill, int32_t* out_tokens, float* out_margins) {
    orc_state* s = orc_state_new(m);
    if (n_prompt > 1 && batched_prefill) {
        orc_forward_batch(m, s, prompt, n_prompt, 0);
    } else {
        for (int t = 0; t < n_prompt; t++) orc_forward_token(m, s, prompt[t], t);
    }
    int n_past = n_prompt;
    int next = orc_argmax(s->logits, m->n_vocab);
    float margin = orc_top2_margin(s->logits, m->n_vocab);
    int n = 0;
    for (int step = 0; step < n_gen; step++) {
        if (n_past >= m->n_ctx) break;
        out_tokens[n] = next;
        if (out_margins) out_margins[n] = margin;
        n++;
        orc_forward_token(m, s, next, n_past);
        n_past++;
        next = orc_argmax(s->logits, m->n_vocab);
        margin = orc_top2_margin(s->logits, m->n_vocab);
    }
    orc_state_free(s);
    return n;
}
