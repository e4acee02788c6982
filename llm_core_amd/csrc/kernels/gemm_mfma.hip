// gemm_mfma.hip — Q4_K x Q8_0 small-M GEMM on the CDNA4 matrix cores.
//
//   Y[t*rows + o] = sum_b sum_s ( d[o,b]*sc[o,b,s]*dx[t,b,s]*S[o,t,b,s]
//                                 - dmin[o,b]*m[o,b,s]*dx[t,b,s]*bsum[t,b,s] )
//
// where S = sum of q4*x8 over one 32-element sub-block (an exact int32) and
// bsum = sum of the sub-block's x8: the per-(row, token) expression
// ds*dq*dot - ms*(dq*sum) of gemm_q4k_q8_avx2_range
// (src/backend/cpu_x86/kernels/gemv_q4k_q8_avx2.cpp:257-346, called from
// gemm_wt_q8, src/models/llama_model.cpp:837-879), restated for a tile of
// 16 rows x 16 tokens.  Y is token-major like the reference's.
//
// A prep kernel re-lays the Q8_0 activations so that a 16-token fragment is
// one contiguous 512-byte load and precomputes dx*bsum.  Then per (16-row,
// 16-token, sub-block) tile one wave issues
//   v_mfma_i32_16x16x32_i8   A = weight nibbles, B = int8 activations  -> S
// scaled on the VALU by sc (24-bit integer multiply) and dx (fp32 FMA), and per
// 256-element block two v_mfma_f32_16x16x4_f32 fold the min term
// (A = dmin*m per row and sub-block, B = dx*bsum per sub-block and token).
// The integer parts are exact; the float combination differs from the scalar
// dot only in summation order.
//
// MFMA operand layout (16x16xK, wave64): A lane l holds row l%16, k-group
// l/16; B lane l holds column l%16, k-group l/16; result lane l holds rows
// 4*(l/16)+i (i = 0..3) of column l%16.  Within a k-group any element order
// works as long as A and B agree; both use natural order here.
//
// Work split: a workgroup owns a (16*RT rows) x (16*TT tokens) tile; its waves
// split the Q4_K blocks of the rows between them and their partial tiles are
// summed in a fixed order in LDS (deterministic results).
#include "common.hpp"

namespace axf {

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

namespace {

constexpr int kTile = 16;  // MFMA tile edge (rows and tokens)

// Activation re-layout for the matrix cores.  XQ8 holds T rows of nkb Q8_0
// records (fp32 d + 32 int8).  Written, for every record kb and token slot
// t < Tp (slots past T are zero):
//   xs [kb][t][32]  the int8 values   (a 16-token fragment is 512 contiguous bytes)
//   dxs[kb][t]      d
//   gxs[kb][t]      d * (sum of the 32 int8), the dq*sum factor of the min term
__global__ __launch_bounds__(256) void k_gemm_prep(const uint8_t* __restrict__ XQ8, int T, int Tp,
                                                   int nkb, uint8_t* __restrict__ xs,
                                                   float* __restrict__ dxs,
                                                   float* __restrict__ gxs) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;  // kb * Tp + t
    if (i >= (long)nkb * Tp) return;
    const int t = (int)(i % Tp), kb = (int)(i / Tp);
    uint4 q0 = make_uint4(0u, 0u, 0u, 0u), q1 = q0;
    float d = 0.f;
    int bs = 0;
    if (t < T) {
        const uint8_t* p = XQ8 + ((size_t)t * nkb + kb) * Q8_0_BYTES;
        d = __uint_as_float(ld4(p));
        q0 = make_uint4(ld4(p + 4), ld4(p + 8), ld4(p + 12), ld4(p + 16));
        q1 = make_uint4(ld4(p + 20), ld4(p + 24), ld4(p + 28), ld4(p + 32));
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int k = 0; k < 8; k++) bs = dot4((int)w[k], 0x01010101, bs);
    }
    uint4* o = reinterpret_cast<uint4*>(xs + (size_t)i * 32);
    o[0] = q0;
    o[1] = q1;
    dxs[i] = d;
    gxs[i] = d * (float)bs;
}

__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) {
    return (long)(((uint64_t)hi << 32) | lo);
}

// Workgroup = NW waves on one (16*RT rows) x (16*TT tokens) tile; wave w takes
// the Q4_K blocks w, w+NW, ... of the rows and the partial tiles are summed in
// a fixed order in LDS.  grid = (row tiles, token tiles); Tp % (16*TT) == 0.
template <int NW, int RT, int TT>
__global__ __launch_bounds__(NW * 64) void k_gemm_mfma_q4k(
    float* __restrict__ Y, const uint8_t* __restrict__ W, const uint8_t* __restrict__ xs,
    const float* __restrict__ dxs, const float* __restrict__ gxs, int rows, int nb,
    long row_bytes, int T, int Tp) {
    __shared__ v4f_t red[NW > 1 ? NW - 1 : 1][RT * TT][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, g = lane >> 4;
    const int row_base = blockIdx.x * (kTile * RT);
    const int tok_base = blockIdx.y * (kTile * TT);
    // uniform bases + 32-bit lane offsets; rows past the end are computed on
    // clamped (valid) data and never stored, token slots past T hold zeros
    const uint8_t* wbase = W + (long)row_base * row_bytes;
    uint32_t wo[RT];
#pragma unroll
    for (int r = 0; r < RT; r++)
        wo[r] = (uint32_t)(min(row_base + kTile * r + col, rows - 1) - row_base) *
                (uint32_t)row_bytes;
    const uint32_t xo = (uint32_t)(tok_base + col) * 32u + 8u * (uint32_t)g;
    const uint32_t kb_stride = (uint32_t)Tp * 32u;

    const v4i_t zi = {0, 0, 0, 0};
    v4f_t acc[RT][TT], macc[RT][TT];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int t = 0; t < TT; t++) {
            acc[r][t] = v4f_t{0.f, 0.f, 0.f, 0.f};
            macc[r][t] = v4f_t{0.f, 0.f, 0.f, 0.f};
        }

    for (int b = wave; b < nb; b += NW) {
        uint4 h[RT];
        uint32_t q[RT][4][2];
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const uint8_t* blk = wbase + (uint32_t)b * Q4K_BYTES + wo[r];
            h[r] = ld16(blk);
#pragma unroll
            for (int p = 0; p < 4; p++) {
                q[r][p][0] = ld4(blk + 16 + 32 * p + 8 * g);
                q[r][p][1] = ld4(blk + 20 + 32 * p + 8 * g);
            }
        }
        const uint8_t* xsb = xs + (size_t)b * 8 * kb_stride;
        const float* dxb = dxs + (size_t)b * 8 * Tp + tok_base + col;
        const float* gxb = gxs + (size_t)b * 8 * Tp + tok_base + col;
        uint32_t xb[TT][8][2];
        float dx[TT][8], gx[TT][2];
#pragma unroll
        for (int t = 0; t < TT; t++) {
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const uint8_t* xp = xsb + s * kb_stride + xo + t * (kTile * 32);
                xb[t][s][0] = ld4(xp);
                xb[t][s][1] = ld4(xp + 4);
                dx[t][s] = dxb[s * Tp + t * kTile];
            }
            gx[t][0] = gxb[g * Tp + t * kTile];
            gx[t][1] = gxb[(4 + g) * Tp + t * kTile];
        }
        // all of the block's loads are in flight before the first use
        __builtin_amdgcn_sched_barrier(0);

#pragma unroll
        for (int r = 0; r < RT; r++) {
            // this lane's weight row (col of tile r): 6-bit scales and mins
            const float d = h2f(h[r].x & 0xffffu), dmin = h2f(h[r].x >> 16);
            const uint32_t sc03 = h[r].y & 0x3f3f3f3fu;
            const uint32_t sc47 = (h[r].w & 0x0f0f0f0fu) | ((h[r].y >> 2) & 0x30303030u);
            const uint32_t m03 = h[r].z & 0x3f3f3f3fu;
            const uint32_t m47 = ((h[r].w >> 4) & 0x0f0f0f0fu) | ((h[r].z >> 2) & 0x30303030u);
            // min-term A operand: row col, sub-blocks g and 4+g
            const float am0 = dmin * (float)((m03 >> (8 * g)) & 0xffu);
            const float am1 = dmin * (float)((m47 >> (8 * g)) & 0xffu);
            // result-side scales: rows 4g+i live in lanes 4g+i
            uint32_t rs03[4], rs47[4];
            float rd[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int src = 4 * g + i;
                rs03[i] = (uint32_t)__shfl((int)sc03, src);
                rs47[i] = (uint32_t)__shfl((int)sc47, src);
                rd[i] = __shfl(d, src);
            }
#pragma unroll
            for (int t = 0; t < TT; t++) {
                v4f_t accb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < 8; s++) {
                    const uint32_t* qp = q[r][s >> 1];
                    const int sh = (s & 1) * 4;
                    const long a =
                        pack2((qp[0] >> sh) & 0x0f0f0f0fu, (qp[1] >> sh) & 0x0f0f0f0fu);
                    const long bx = pack2(xb[t][s][0], xb[t][s][1]);
                    const v4i_t c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bx, zi, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        // |S| < 2^17 and sc < 64: the 24-bit multiply is exact
                        const int scv =
                            (int)(((s < 4 ? rs03[i] : rs47[i]) >> (8 * (s & 3))) & 0xffu);
                        accb[i] = fmaf((float)__mul24(c[i], scv), dx[t][s], accb[i]);
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; i++) acc[r][t][i] = fmaf(rd[i], accb[i], acc[r][t][i]);
                macc[r][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(am0, gx[t][0], macc[r][t], 0, 0, 0);
                macc[r][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(am1, gx[t][1], macc[r][t], 0, 0, 0);
            }
        }
    }

#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int t = 0; t < TT; t++) {
            acc[r][t] -= macc[r][t];
            if (NW > 1 && wave > 0) red[wave - 1][r * TT + t][lane] = acc[r][t];
        }
    if (NW > 1) __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int t = 0; t < TT; t++) {
                v4f_t v = acc[r][t];
#pragma unroll
                for (int w = 0; w < NW - 1; w++) v += red[w][r * TT + t][lane];
                const int tok = tok_base + kTile * t + col;
                if (tok < T) {
                    float* yr = Y + (size_t)tok * rows;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int o = row_base + kTile * r + 4 * g + i;
                        if (o < rows) yr[o] = v[i];
                    }
                }
            }
    }
}

struct MfmaCfg {
    int nw, rt, tt;
};

MfmaCfg pick_mfma(int T, int nb) {
    const int nw = nb >= 8 ? 8 : 4;
    return {nw, 2, T > kTile ? 2 : 1};
}

int padded_tokens(int T, const MfmaCfg& c) {
    const int q = kTile * c.tt;
    return (T + q - 1) / q * q;
}

template <int NW, int RT, int TT>
void launch_cfg(float* Y, const uint8_t* W, const uint8_t* xs, const float* dxs,
                const float* gxs, int rows, int nb, long row_bytes, int T, int Tp,
                hipStream_t st) {
    const dim3 grid((unsigned)((rows + kTile * RT - 1) / (kTile * RT)),
                    (unsigned)(Tp / (kTile * TT)));
    hipLaunchKernelGGL((k_gemm_mfma_q4k<NW, RT, TT>), grid, dim3(NW * 64), 0, st, Y, W, xs, dxs,
                       gxs, rows, nb, row_bytes, T, Tp);
}

}  // namespace

size_t gemm_mfma_scratch_bytes(int T, int nb) {
    if (T <= 0 || nb <= 0) return 0;
    const size_t tp = (size_t)padded_tokens(T, pick_mfma(T, nb));
    return (size_t)nb * 8 * tp * (32 + 4 + 4);
}

hipError_t launch_gemm_mfma_q4k_q8(float* Y, const void* W, const void* XQ8, int rows, int T,
                                   int nb, long row_bytes, void* scratch, hipStream_t st) {
    if (rows <= 0 || T <= 0 || nb <= 0 || scratch == nullptr) return hipErrorInvalidValue;
    const MfmaCfg c = pick_mfma(T, nb);
    const int Tp = padded_tokens(T, c);
    const int nkb = nb * 8;
    // 32-bit lane offsets: a weight tile and the re-laid activation must each
    // span < 4 GiB
    if ((uint64_t)row_bytes * kTile * c.rt >= (1ull << 32) ||
        (uint64_t)nkb * Tp * 32 >= (1ull << 32))
        return hipErrorInvalidValue;
    auto* xs = static_cast<uint8_t*>(scratch);
    auto* dxs = reinterpret_cast<float*>(xs + (size_t)nkb * Tp * 32);
    auto* gxs = dxs + (size_t)nkb * Tp;
    const long n = (long)nkb * Tp;
    hipLaunchKernelGGL(k_gemm_prep, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       static_cast<const uint8_t*>(XQ8), T, Tp, nkb, xs, dxs, gxs);
    const auto* w = static_cast<const uint8_t*>(W);
#define AXF_MFMA_CASE(NW, RT, TT)                                                          \
    if (c.nw == NW && c.rt == RT && c.tt == TT)                                            \
        launch_cfg<NW, RT, TT>(Y, w, xs, dxs, gxs, rows, nb, row_bytes, T, Tp, st);        \
    else
    AXF_MFMA_CASE(8, 2, 2)
    AXF_MFMA_CASE(8, 2, 1)
    AXF_MFMA_CASE(4, 2, 2)
    AXF_MFMA_CASE(4, 2, 1)
    return hipErrorInvalidValue;
#undef AXF_MFMA_CASE
    return hipGetLastError();
}

}  // namespace axf
