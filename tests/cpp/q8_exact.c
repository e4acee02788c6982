/* q8_exact.c - checks two shortcuts of the device Q8_0 quantiser (q8_quant4
 * in llm_core_amd/csrc/kernels/common.hpp) against the plain formula of the
 * reference's quantize_q8_avx2 (d = amax/127, q = rint(v * 127/amax) saturated
 * to int8, quant_q8_avx2.cpp:33-84):
 *   1. div127: amax/127 as  q0 = amax*RN(1/127); r = fma(-q0, 127, amax);
 *      fma(r, RN(1/127), q0)  - every non-negative finite float, exhaustively;
 *   2. the int8 of rint(RN(v*id)) read as the low byte of RN(RN(v*id) + 1.5*2^23),
 *      without saturation - random blocks of several magnitudes, blocks whose
 *      products land on and next to halves, amax = 0, and tiny blocks whose
 *      127/amax overflows (every value -128, as cvtps_epi32 + packs).
 * Built with -ffp-contract=off so that products and sums round as written.
 * Prints "ok" and exits 0, or prints the first mismatch and exits 1. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float fbits(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static uint32_t bitsf(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }

static float div127(float a) {
    const float y = 1.0f / 127.0f;
    const float q0 = a * y;
    const float r = fmaf(-q0, 127.0f, a);
    return fmaf(r, y, q0);
}

static uint32_t lcg(uint64_t* s) { *s = *s * 6364136223846793005ull + 1442695040888963407ull; return (uint32_t)(*s >> 33); }

/* reference and shortcut quantisation of one block; returns 0 when equal.
 * The reference's _mm256_cvtps_epi32 gives INT_MIN for a product that is not
 * a finite int32 (the packs then give -128): with 0 < amax < 127/FLT_MAX the
 * reciprocal overflows to +inf and every product is +-inf or NaN.  The
 * shortcut selects -128 for the whole block when id is infinite. */
static int block_check(const float* v) {
    float amax = 0.f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    const float id = amax > 0.f ? 127.f / amax : 0.f;
    if (div127(amax) != amax / 127.f) return 1;
    for (int i = 0; i < 32; i++) {
        const float pr = v[i] * id;
        uint8_t want;
        if (!(fabsf(pr) < 2147483648.f)) {
            want = 0x80;
        } else {
            float r = rintf(pr);
            r = fminf(fmaxf(r, -128.f), 127.f);
            want = (uint8_t)((int)r & 0xff);
        }
        const float p = v[i] * id;
        const uint8_t got = isinf(id) ? 0x80 : (uint8_t)(bitsf(p + 12582912.f) & 0xff);
        if (want != got) {
            printf("block mismatch: v=%a id=%a want %d got %d\n", v[i], id, (int8_t)want, (int8_t)got);
            return 1;
        }
    }
    return 0;
}

int main(void) {
    long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long hi = 0; hi < 0x7f80; hi++) {
        for (uint32_t lo = 0; lo < 0x10000; lo++) {
            const float a = fbits(((uint32_t)hi << 16) | lo);
            if (div127(a) != a / 127.0f) bad++;
        }
    }
    if (bad) { printf("div127: %ld mismatches\n", bad); return 1; }

    uint64_t s = 12345;
    float v[32];
    for (int t = 0; t < 2000000; t++) {
        const float scale = ldexpf(1.f, (int)(lcg(&s) % 80) - 40);
        for (int i = 0; i < 32; i++) v[i] = ((float)(lcg(&s) & 0xffffff) / 8388608.f - 1.f) * scale;
        if (t % 4 == 1) v[lcg(&s) % 32] = 0.f;
        if (block_check(v)) return 1;
    }
    /* products on and next to halves: amax = 127 gives id = 1, v = k + 0.5 and neighbours */
    for (int k = -127; k < 127; k++) {
        for (int d = -2; d <= 2; d++) {
            for (int i = 0; i < 32; i++) v[i] = 0.f;
            v[0] = 127.f;
            v[1] = fbits(bitsf((float)k + 0.5f) + d);
            v[2] = -v[1];
            if (block_check(v)) return 1;
        }
    }
    for (int i = 0; i < 32; i++) v[i] = 0.f;
    if (block_check(v)) return 1;
    /* tiny blocks: amax around 127/FLT_MAX (id overflows below it), subnormal
     * values, and zeros beside them */
    const float lim = 127.f / 3.40282347e38f;
    const float tiny[] = {lim, nextafterf(lim, 0.f), nextafterf(lim, 1.f), lim * 0.5f,
                          1.17549435e-38f, 1e-39f, 1.4e-45f, 2.8e-45f};
    for (unsigned t = 0; t < sizeof tiny / sizeof tiny[0]; t++) {
        for (int i = 0; i < 32; i++) v[i] = (i % 3 == 0) ? 0.f : (i % 3 == 1 ? tiny[t] : -tiny[t] * 0.5f);
        if (block_check(v)) return 1;
    }
    printf("ok\n");
    return 0;
}
