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
// one contiguous 512-byte block and precomputes dx*bsum.  The GEMM kernel then
// streams the K dimension one Q4_K block (256 weights per row) at a time
// through an S-deep ring of LDS stages, each filled by global_load_lds_dwordx4
// copies (1 KiB per wave instruction, no VGPR staging): the workgroup's weight
// rows, the tokens' int8 values, dx and dx*bsum.  Per (16-token, 16-row,
// sub-block) tile one wave issues
//   v_mfma_i32_16x16x32_i8   A = int8 activations, B = weight nibbles  -> S
// scaled on the VALU by sc (24-bit integer multiply) and dx (fp32 FMA), and per
// block two v_mfma_f32_16x16x4_f32 fold the min term (A = dx*bsum per token
// and sub-block, B = dmin*m per sub-block and weight row).  The integer parts
// are exact; the float combination differs from the scalar dot only in
// summation order.
//
// MFMA operand layout (16x16xK, wave64): A lane l holds row l%16, k-group
// l/16; B lane l holds column l%16, k-group l/16; result lane l holds rows
// 4*(l/16)+i (i = 0..3) of column l%16.  Within a k-group any element order
// works as long as A and B agree; both use natural order here.  With tokens
// as A's rows and weight rows as B's columns, every weight-side scale of a
// result lane belongs to that lane's own weight row.
//
// Work split: a workgroup owns a (16*RT rows) x (16*TT tokens) tile; each wave
// takes whole 16x16 tiles, or, when there are fewer tiles than waves, a
// subset of the sub-blocks of one tile, whose partial tiles are then summed in
// a fixed order in LDS (deterministic results).
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

typedef __attribute__((address_space(1))) const void gmem_t;
typedef __attribute__((address_space(3))) void lmem_t;

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] bits 3:0,
// vmcnt[5:4] bits 15:14, expcnt and lgkmcnt at their maxima)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// One K-chunk (one Q4_K block, 256 weights per row) as staged in LDS:
//   [RW rows][144 B] weights | [8 records][TW tokens][32 B] int8 activations |
//   [8][TW] dx | [8][TW] dx*bsum.
// It is copied by 1 KiB pieces (64 lanes x 16 B, global_load_lds_dwordx4);
// wave w copies pieces w, w+NW, ...
template <int RT, int TT, int NW, int S>
struct Stage {
    static constexpr int RW = kTile * RT, TW = kTile * TT;
    static constexpr int WB = RW * Q4K_BYTES;
    static constexpr int XB = 8 * TW * 32;
    static constexpr int DB = 8 * TW * 4;
    static constexpr int BYTES = WB + XB + 2 * DB;
    static constexpr int PIECES = (BYTES + 1023) / 1024;
    static constexpr int ALLOC = PIECES * 1024;
    static constexpr int PMAX = (PIECES + NW - 1) / NW;  // pieces of the busiest wave
    static constexpr int PMIN = PIECES / NW;             // pieces of every wave
    static constexpr int NTILE = RT * TT;
    static constexpr int WT = NTILE >= NW ? NTILE / NW : 1;  // tiles per wave
    static constexpr int KS = NTILE >= NW ? 1 : NW / NTILE;  // waves per tile (sub-block split)
    static_assert(WB % 16 == 0 && XB % 1024 == 0 && DB % 16 == 0, "piece alignment");
    static_assert(NTILE % NW == 0 || NW % NTILE == 0, "tile split");
    static_assert(TT % WT == 0 && 8 % KS == 0, "tile split");
};

// The sub-blocks s = KPH, KPH+KS, ... of one staged chunk for this wave's
// tiles.  MFMA operands: A = 16 tokens (row l%16 of A is token col), B = 16
// weight rows (column l%16 is weight row col), so result lane l holds tokens
// 4g+i of weight row col: every weight-side scale is lane-local.  All LDS
// reads are issued first, then the MFMAs back to back, then the scaling
// (integer sc via a 24-bit multiply, dx via an fp32 FMA).
template <class G, int KPH>
__device__ __forceinline__ void mfma_sub_blocks(const uint8_t* wl, const uint8_t* xl,
                                                const float* dl, int g, int col, int tt0,
                                                uint32_t sc03, uint32_t sc47,
                                                v4f_t (&accb)[G::WT]) {
    constexpr int TW = G::TW, NS = 8 / G::KS;
    const v4i_t zi = {0, 0, 0, 0};
    uint2 qv[4];
#pragma unroll
    for (int p = 0; p < 4; p++) qv[p] = *reinterpret_cast<const uint2*>(wl + 16 + 32 * p + 8 * g);
    uint2 xv[G::WT][NS];
    float4 dx[G::WT][NS];
#pragma unroll
    for (int w = 0; w < G::WT; w++)
#pragma unroll
        for (int sj = 0; sj < NS; sj++) {
            const int s = KPH + G::KS * sj;
            const int tok = kTile * (tt0 + w);
            xv[w][sj] = *reinterpret_cast<const uint2*>(xl + (s * TW + tok + col) * 32 + 8 * g);
            dx[w][sj] = *reinterpret_cast<const float4*>(dl + s * TW + tok + 4 * g);
        }
    v4i_t c[G::WT][NS];
#pragma unroll
    for (int sj = 0; sj < NS; sj++) {
        const int s = KPH + G::KS * sj;
        const int sh = (s & 1) * 4;
        const long bw = pack2((qv[s >> 1].x >> sh) & 0x0f0f0f0fu, (qv[s >> 1].y >> sh) & 0x0f0f0f0fu);
#pragma unroll
        for (int w = 0; w < G::WT; w++)
            c[w][sj] = __builtin_amdgcn_mfma_i32_16x16x32_i8(pack2(xv[w][sj].x, xv[w][sj].y), bw,
                                                             zi, 0, 0, 0);
    }
#pragma unroll
    for (int sj = 0; sj < NS; sj++) {
        const int s = KPH + G::KS * sj;
        const int scv = (int)(((s < 4 ? sc03 : sc47) >> (8 * (s & 3))) & 0xffu);
#pragma unroll
        for (int w = 0; w < G::WT; w++) {
            // |S| < 2^17 and sc < 64: the 24-bit multiply is exact
            accb[w][0] = fmaf((float)__mul24(c[w][sj][0], scv), dx[w][sj].x, accb[w][0]);
            accb[w][1] = fmaf((float)__mul24(c[w][sj][1], scv), dx[w][sj].y, accb[w][1]);
            accb[w][2] = fmaf((float)__mul24(c[w][sj][2], scv), dx[w][sj].z, accb[w][2]);
            accb[w][3] = fmaf((float)__mul24(c[w][sj][3], scv), dx[w][sj].w, accb[w][3]);
        }
    }
}

// One step of the K loop (inlined): copy chunk `bnext` into `nxt`, then, for
// i >= 0, wait for chunk i and compute it from `cur`.
template <int RT, int TT, int NW, int S>
__device__ __forceinline__ void gemm_step(
    const uint8_t* __restrict__ cur, uint8_t* __restrict__ nxt, bool do_copy, int bnext, int i,
    int nb, const uint8_t* const (&src)[Stage<RT, TT, NW, S>::PMAX],
    const uint32_t (&step)[Stage<RT, TT, NW, S>::PMAX], int wave, int lane, int col, int g,
    int kph, int tt0, int wrow, v4f_t (&acc)[Stage<RT, TT, NW, S>::WT],
    v4f_t (&macc)[Stage<RT, TT, NW, S>::WT]) {
    using G = Stage<RT, TT, NW, S>;
    constexpr int TW = G::TW;
    if (do_copy) {
#pragma unroll
        for (int j = 0; j < G::PMAX; j++) {
            if (wave + NW * j < G::PIECES)
                __builtin_amdgcn_global_load_lds((gmem_t*)(src[j] + (size_t)bnext * step[j]),
                                                 (lmem_t*)(nxt + (wave + NW * j) * 1024), 16, 0,
                                                 0);
        }
    }
    if (i < 0) return;
        // own copies of chunk i done (at most min(S-1, nb-1-i) later chunks in flight)
        const int later = min(S - 1, nb - 1 - i);
        if constexpr (S >= 4) {
            if (later >= 3) wait_vmcnt<3 * G::PMIN>();
            else if (later == 2) wait_vmcnt<2 * G::PMIN>();
            else if (later == 1) wait_vmcnt<G::PMIN>();
            else wait_vmcnt<0>();
        } else {
            if (later >= 2) wait_vmcnt<2 * G::PMIN>();
            else if (later == 1) wait_vmcnt<G::PMIN>();
            else wait_vmcnt<0>();
        }
        // every wave's copies of chunk i are in LDS (a bare barrier: the
        // fence of __syncthreads would also wait for the later chunks)
        __builtin_amdgcn_s_barrier();

        const uint8_t* stg = cur;
        const uint8_t* wl = stg + wrow;
        const uint8_t* xl = stg + G::WB;
        const float* dl = reinterpret_cast<const float*>(stg + G::WB + G::XB);
        const float* gl = dl + 8 * TW;

        // this lane's weight row (col of the wave's row tile): scales and mins
        const uint4 h = *reinterpret_cast<const uint4*>(wl);
        const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
        const uint32_t sc03 = h.y & 0x3f3f3f3fu;
        const uint32_t sc47 = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
        v4f_t accb[G::WT];
#pragma unroll
        for (int w = 0; w < G::WT; w++) accb[w] = v4f_t{0.f, 0.f, 0.f, 0.f};
        // sub-blocks of this wave's phase, the phase a compile-time constant
        if (kph == 0) mfma_sub_blocks<G, 0>(wl, xl, dl, g, col, tt0, sc03, sc47, accb);
        if constexpr (G::KS > 1) {
            if (kph == 1) mfma_sub_blocks<G, 1>(wl, xl, dl, g, col, tt0, sc03, sc47, accb);
        }
        if constexpr (G::KS > 2) {
            if (kph == 2) mfma_sub_blocks<G, 2>(wl, xl, dl, g, col, tt0, sc03, sc47, accb);
            if (kph == 3) mfma_sub_blocks<G, 3>(wl, xl, dl, g, col, tt0, sc03, sc47, accb);
        }
#pragma unroll
        for (int w = 0; w < G::WT; w++) {
#pragma unroll
            for (int ii = 0; ii < 4; ii++) acc[w][ii] = fmaf(d, accb[w][ii], acc[w][ii]);
        }
        if (kph == 0) {
            // min term: A = dq*sum (token col, sub-blocks g / 4+g), B = dmin*m
            // (weight row col, the same sub-blocks)
            const uint32_t m03 = h.z & 0x3f3f3f3fu;
            const uint32_t m47 = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
            const float am0 = dmin * (float)((m03 >> (8 * g)) & 0xffu);
            const float am1 = dmin * (float)((m47 >> (8 * g)) & 0xffu);
#pragma unroll
            for (int w = 0; w < G::WT; w++) {
                const int tok = kTile * (tt0 + w) + col;
                macc[w] = __builtin_amdgcn_mfma_f32_16x16x4f32(gl[g * TW + tok], am0, macc[w], 0, 0, 0);
                macc[w] = __builtin_amdgcn_mfma_f32_16x16x4f32(gl[(4 + g) * TW + tok], am1, macc[w], 0, 0, 0);
            }
        }
        // stage u is free for chunk i + S (its reads were consumed above)
        __builtin_amdgcn_s_barrier();
}

// Workgroup = NW waves on a (16*RT rows) x (16*TT tokens) tile; the K loop
// streams one Q4_K block per step through an S-deep ring of LDS stages.
// grid = (row tiles, token tiles); Tp % (16*TT) == 0.
template <int RT, int TT, int NW, int S>
__global__ __launch_bounds__(NW * 64) void k_gemm_mfma_q4k(
    float* __restrict__ Y, const uint8_t* __restrict__ W, const uint8_t* __restrict__ xs,
    const float* __restrict__ dxs, const float* __restrict__ gxs, int rows, int nb,
    long row_bytes, int T, int Tp) {
    using G = Stage<RT, TT, NW, S>;
    constexpr int RW = G::RW, TW = G::TW;
    __shared__ __attribute__((aligned(16))) uint8_t smem[S * G::ALLOC];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, g = lane >> 4;
    const int row_base = blockIdx.x * RW;
    const int tok_base = blockIdx.y * TW;

    // ---- copy plan: per piece this lane's source (chunk 0) and its step per chunk
    const uint8_t* src[G::PMAX];
    uint32_t step[G::PMAX];
#pragma unroll
    for (int j = 0; j < G::PMAX; j++) {
        int o = (wave + NW * j) * 1024 + lane * 16;
        if (o >= G::BYTES) o = 0;  // tail of the last piece: a harmless duplicate
        if (o < G::WB) {
            const int r = o / Q4K_BYTES;
            src[j] = W + (long)min(row_base + r, rows - 1) * row_bytes + (o - r * Q4K_BYTES);
            step[j] = Q4K_BYTES;
        } else if (o < G::WB + G::XB) {
            const int x = o - G::WB, k = x / (TW * 32);
            src[j] = xs + ((size_t)k * Tp + tok_base) * 32 + (x - k * TW * 32);
            step[j] = 8u * (uint32_t)Tp * 32u;
        } else {
            const int y = o - G::WB - G::XB;
            const int which = y / G::DB, z = y - which * G::DB, k = z / (TW * 4);
            const float* base = which == 0 ? dxs : gxs;
            src[j] = reinterpret_cast<const uint8_t*>(base + (size_t)k * Tp + tok_base) +
                     (z - k * TW * 4);
            step[j] = 8u * (uint32_t)Tp * 4u;
        }
    }
    // ---- this wave's tiles and sub-blocks
    const int tg = wave % (NW / G::KS);     // tile group
    const int kph = wave / (NW / G::KS);    // sub-block phase
    const int t0 = tg * G::WT;              // first tile (tile = rt*TT + tt)
    const int rt = t0 / TT, tt0 = t0 % TT;
    const int wrow = (kTile * rt + col) * Q4K_BYTES;

    v4f_t acc[G::WT], macc[G::WT];
#pragma unroll
    for (int w = 0; w < G::WT; w++) {
        acc[w] = v4f_t{0.f, 0.f, 0.f, 0.f};
        macc[w] = v4f_t{0.f, 0.f, 0.f, 0.f};
    }

    // Step i copies chunk i+S-1 and (from i = 0) computes chunk i.  Every
    // copy is issued by the same instruction inside gemm_step, whose stage
    // pointers are __restrict__: the copy target and the stage being read are
    // distinct, so the compiler adds no wait for the copies in flight before
    // the LDS reads; the explicit vmcnt wait orders chunk i itself.
    for (int i = 1 - S; i < nb; i++) {
        const int inext = i + S - 1;
        gemm_step<RT, TT, NW, S>(smem + ((i + S) % S) * G::ALLOC, smem + (inext % S) * G::ALLOC,
                                 inext < nb, inext, i, nb, src, step, wave, lane, col, g, kph,
                                 tt0, wrow, acc, macc);
    }

    // ---- sum the KS sub-block phases of each tile (fixed order), store
    v4f_t* red = reinterpret_cast<v4f_t*>(smem);
    if constexpr (G::KS > 1) {
        if (kph > 0) {
#pragma unroll
            for (int w = 0; w < G::WT; w++)
                red[((kph - 1) * (NW / G::KS) + tg) * G::WT * 64 + w * 64 + lane] = acc[w] - macc[w];
        }
        __syncthreads();
    }
    if (kph == 0) {
#pragma unroll
        for (int w = 0; w < G::WT; w++) {
            v4f_t v = acc[w] - macc[w];
#pragma unroll
            for (int k = 1; k < G::KS; k++) v += red[((k - 1) * (NW / G::KS) + tg) * G::WT * 64 + w * 64 + lane];
            const int o = row_base + kTile * rt + col;
            if (o < rows) {
#pragma unroll
                for (int ii = 0; ii < 4; ii++) {
                    const int tok = tok_base + kTile * (tt0 + w) + 4 * g + ii;
                    if (tok < T) Y[(size_t)tok * rows + o] = v[ii];
                }
            }
        }
    }
}

struct MfmaCfg {
    int rt, tt;
};

MfmaCfg pick_mfma(int T, int nb) {
    (void)nb;
    if (T <= 16) return {2, 1};
    return {2, T > 32 ? 4 : 2};
}

int padded_tokens(int T, const MfmaCfg& c) {
    const int q = kTile * c.tt;
    return (T + q - 1) / q * q;
}

template <int RT, int TT, int NW, int S>
void launch_cfg(float* Y, const uint8_t* W, const uint8_t* xs, const float* dxs,
                const float* gxs, int rows, int nb, long row_bytes, int T, int Tp,
                hipStream_t st) {
    const dim3 grid((unsigned)((rows + kTile * RT - 1) / (kTile * RT)),
                    (unsigned)(Tp / (kTile * TT)));
    hipLaunchKernelGGL((k_gemm_mfma_q4k<RT, TT, NW, S>), grid, dim3(NW * 64), 0, st, Y, W, xs,
                       dxs, gxs, rows, nb, row_bytes, T, Tp);
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
#define AXF_MFMA_CASE(RT, TT, NW, S)                                                       \
    if (c.rt == RT && c.tt == TT)                                                          \
        launch_cfg<RT, TT, NW, S>(Y, w, xs, dxs, gxs, rows, nb, row_bytes, T, Tp, st);     \
    else
    AXF_MFMA_CASE(2, 1, 4, 4)
    AXF_MFMA_CASE(2, 2, 4, 4)
    AXF_MFMA_CASE(2, 4, 8, 3)
    return hipErrorInvalidValue;
#undef AXF_MFMA_CASE
    return hipGetLastError();
}

}  // namespace axf
