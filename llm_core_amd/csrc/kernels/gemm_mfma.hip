// gemm_mfma.hip — Q4_K x Q8_0 and Q6_K x Q8_0 small-M GEMMs on the CDNA4 matrix
// cores (the fp16 Q4_K kernel for 65+ tokens and the Q6_K kernel are described
// where they start, below).
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
    int b0 = 0, b1 = 0;
    if (t < T) {
        const uint8_t* p = XQ8 + ((size_t)t * nkb + kb) * Q8_0_BYTES;
        d = __uint_as_float(ld4(p));
        q0 = make_uint4(ld4(p + 4), ld4(p + 8), ld4(p + 12), ld4(p + 16));
        q1 = make_uint4(ld4(p + 20), ld4(p + 24), ld4(p + 28), ld4(p + 32));
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            b0 = dot4((int)w[k], 0x01010101, b0);
            b1 = dot4((int)w[k + 4], 0x01010101, b1);
        }
    }
    uint4* o = reinterpret_cast<uint4*>(xs + (size_t)i * 32);
    o[0] = q0;
    o[1] = q1;
    dxs[i] = d;
    gxs[i] = d * (float)(b0 + b1);
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

// Wait until at most `later` chunks of P copies each are still in flight
// (later <= L): s_waitcnt vmcnt(later * P) with the count a constant.
template <int P, int L>
__device__ __forceinline__ void wait_later(int later) {
    if constexpr (L == 0) {
        wait_vmcnt<0>();
    } else {
        if (later >= L) wait_vmcnt<L * P>();
        else wait_later<P, L - 1>(later);
    }
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
    static_assert((KS - 1) * (NW / KS) * WT * 64 * 16 <= S * ALLOC, "reduction space");
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
            xv[w][sj] = *reinterpret_cast<const uint2*>(
                xl + (s * TW + tok + col) * 32 + 8 * (g ^ (2 * ((col >> 3) & 1))));
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
        wait_later<G::PMIN, S - 1>(later);
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
        if constexpr (G::KS > 4) {
            if (kph == 4) mfma_sub_blocks<G, 4>(wl, xl, dl, g, col, tt0, sc03, sc47, accb);
            if (kph == 5) mfma_sub_blocks<G, 5>(wl, xl, dl, g, col, tt0, sc03, sc47, accb);
            if (kph == 6) mfma_sub_blocks<G, 6>(wl, xl, dl, g, col, tt0, sc03, sc47, accb);
            if (kph == 7) mfma_sub_blocks<G, 7>(wl, xl, dl, g, col, tt0, sc03, sc47, accb);
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
            // halves of token t swapped when bit 3 of t is set (bank-conflict-free
            // 8-byte reads, as in the Q6_K kernel)
            const int x = o - G::WB, k = x / (TW * 32), r = x - k * TW * 32, t = r >> 5;
            const int hb = ((r >> 4) & 1) ^ ((t >> 3) & 1);
            src[j] = xs + ((size_t)k * Tp + tok_base) * 32 + t * 32 + hb * 16;
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

// ---------------------------------------------------------------------------
// Q4_K x Q8_0 for a few tokens (T <= 64), weights loaded straight into
// registers and no activation re-layout kernel.
//
// Measured on the 25.4 MB 11008x4096 matrix: 16-byte loads that cover 64
// contiguous bytes of each of 16 rows run at the plain-read rate (5.7-5.9 us),
// loads of 8 bytes per lane in the MFMA operand layout do not (8.5 us), and
// every extra vector-memory instruction per wave and block (activation
// fragments, dx) costs about 0.35 us.  So:
//   * a workgroup owns RT row tiles (wave w: 16 rows), a K range of KB
//     blocks (split-K over gridDim.y = ceil(nb / KB) workgroups) and TT
//     token tiles of 16 tokens starting at token 16 * TT * blockIdx.z (the
//     token groups over gridDim.z);
//   * lane (col, g) loads its row's block header and qs bytes 32g..32g+31
//     (chunk g: sub-blocks 2g and 2g+1) as 16-byte loads, all up front;
//     two rounds of v_permlane32_swap / v_permlane16_swap turn "lane g holds
//     chunk g" into "lane g holds bytes 8g..8g+7 of every chunk", the B
//     operand layout of v_mfma_i32_16x16x32_i8;
//   * the workgroup stages its K range of its tokens' activations once, 16
//     tokens at a time, into LDS (per token a contiguous run of Q8_0 records, copied by
//     16-byte loads; one pad chunk per token spreads the tokens over the
//     banks), then derives dx and dx*bsum per (record, token) from it;
//   * per sub-block: one int8 MFMA (A = token x from LDS, B = the nibbles),
//     S*sc by a 24-bit multiply, dx by an fp32 FMA, d per block, the min term
//     by two v_mfma_f32_16x16x4f32 per block, as in the ring kernel above;
//   * the blocks of the K range are computed in order, each as soon as its
//     own loads have arrived (the loop is unrolled; a loop that moved the
//     later blocks' registers down a slot per iteration waited for all of
//     them before the first block's compute ended);
//   * with gridDim.y > 1 each workgroup writes its partial tiles to scratch,
//     and k_gemm_splitk_sum(4) adds them in K order: results are
//     deterministic whatever the finishing order.
// ---------------------------------------------------------------------------
template <int RT, int KB, int TT>
struct Rx {
    static constexpr int CPT = KB * 18;           // 16-B chunks of one token's K range
    static constexpr int TSTR = CPT + 1;          // LDS token stride in chunks (one pad)
    static constexpr int XCH = kTile * TT * TSTR; // chunks staged (all token tiles)
    static constexpr int XP = (XCH + 63) / 64;    // 1 KiB pieces (64 lanes x 16 B)
    static constexpr int XPW = (XP + RT - 1) / RT;
    static constexpr int NS = 8 * KB;             // Q8_0 records per token
};

template <int RT, int KB, int TT>
__global__ __launch_bounds__(RT * 64) void k_gemm_q4k_rx(
    float* __restrict__ Y, const uint8_t* __restrict__ W, const uint8_t* __restrict__ XQ8,
    float* __restrict__ part, int rows, int nb, long row_bytes, int T) {
    using G = Rx<RT, KB, TT>;
    __shared__ __align__(16) uint8_t xl[G::XP * 1024];
    __shared__ __align__(16) float dxl[TT * G::NS * kTile];  // [tile][record][token]
    __shared__ float gxl[TT * G::NS * kTile];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, g = lane >> 4;
    const int S = (int)gridDim.y, ks = (int)blockIdx.y, kb0 = ks * KB;
    const size_t tok_bytes = (size_t)nb * 8 * Q8_0_BYTES;
    // chunks of a token row from record 8*kb0 on (the last K range may be short)
    const int cend = min(G::CPT, (nb - kb0) * 18) - 1;
    const int row0 = ((int)blockIdx.x * RT + wave) * kTile;
    const int o = row0 + col;
    const int t0 = (int)blockIdx.z * kTile * TT;  // first token of this token group

    // activations: slot (u, j) with u = 16*tile + t, j < CPT: chunk j of
    // token t0 + u's K range (tokens past T repeat token T-1).  Issued before
    // the weights, so that they are waited for first.
    uint4 xr[G::XPW];
#pragma unroll
    for (int k = 0; k < G::XPW; k++) {
        const int piece = wave + RT * k;
        if (piece < G::XP) {
            const int slot = piece * 64 + lane;
            const int u = min(slot / G::TSTR, kTile * TT - 1);
            const int j = min(slot - (slot / G::TSTR) * G::TSTR, cend);
            const int tok = min(t0 + u, T - 1);
            xr[k] = ld16(XQ8 + (size_t)tok * tok_bytes + (size_t)kb0 * 8 * Q8_0_BYTES + 16 * j);
        }
    }
    // weights: row o (clamped), blocks kb0.. (clamped; blocks past nb are
    // computed on block nb-1 and their contribution dropped)
    const uint8_t* wr = W + (size_t)min(o, rows - 1) * row_bytes;
    uint4 hdr[KB];
    uint32_t P[KB][4][2];
#pragma unroll
    for (int b = 0; b < KB; b++) {
        const uint8_t* blk = wr + (size_t)min(kb0 + b, nb - 1) * Q4K_BYTES;
        hdr[b] = ld16(blk);
        const uint4 qa = ld16(blk + 16 + 32 * g), qb = ld16(blk + 32 + 32 * g);
        P[b][0][0] = qa.x; P[b][0][1] = qa.y; P[b][1][0] = qa.z; P[b][1][1] = qa.w;
        P[b][2][0] = qb.x; P[b][2][1] = qb.y; P[b][3][0] = qb.z; P[b][3][1] = qb.w;
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < G::XPW; k++) {
        const int piece = wave + RT * k;
        if (piece < G::XP) *reinterpret_cast<uint4*>(xl + piece * 1024 + lane * 16) = xr[k];
    }
    __syncthreads();
    // dx and dx*bsum per (tile, record, token)
    for (int i = threadIdx.x; i < TT * G::NS * kTile; i += RT * 64) {
        const int t = i & (kTile - 1), sr = (i >> 4) % G::NS, w = (i >> 4) / G::NS;
        const uint32_t* rec = reinterpret_cast<const uint32_t*>(
            xl + (kTile * w + t) * G::TSTR * 16 + sr * Q8_0_BYTES);
        const float d = __uint_as_float(rec[0]);
        int sum = 0;
#pragma unroll
        for (int k = 1; k <= 8; k++) sum = dot4((int)rec[k], 0x01010101, sum);
        dxl[i] = d;
        gxl[i] = d * (float)sum;
    }
    __syncthreads();

    const v4i_t zi = {0, 0, 0, 0};
    v4f_t acc[TT], macc[TT];
#pragma unroll
    for (int w = 0; w < TT; w++) acc[w] = macc[w] = v4f_t{0.f, 0.f, 0.f, 0.f};
    // Blocks in order, unrolled: block b's compute waits only for block b's
    // loads (and the earlier ones), so it starts while the later blocks are
    // still arriving.  A scheduling fence between blocks keeps the compiler
    // from building several blocks' operands at once.
#pragma unroll
    for (int b = 0; b < KB; b++) {
        // lane g holds chunk g (pieces 0..3 = bytes 8j..8j+7 of qs 32g..32g+31);
        // afterwards Q[c] = bytes 8g..8g+7 of chunk c
        uint32_t Q[4][2];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const auto r02 = __builtin_amdgcn_permlane32_swap(P[b][0][e], P[b][2][e], false, false);
            const auto r13 = __builtin_amdgcn_permlane32_swap(P[b][1][e], P[b][3][e], false, false);
            const auto r01 = __builtin_amdgcn_permlane16_swap(r02[0], r13[0], false, false);
            const auto r23 = __builtin_amdgcn_permlane16_swap(r02[1], r13[1], false, false);
            Q[0][e] = r01[0]; Q[1][e] = r01[1];
            Q[2][e] = r23[0]; Q[3][e] = r23[1];
        }
        const uint4 h = hdr[b];
        const bool lv = kb0 + b < nb;
        const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
        const uint32_t sc03 = h.y & 0x3f3f3f3fu;
        const uint32_t sc47 = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
        const uint32_t m03 = h.z & 0x3f3f3f3fu;
        const uint32_t m47 = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
        const float am0 = dmin * (float)((m03 >> (8 * g)) & 0xffu);
        const float am1 = dmin * (float)((m47 >> (8 * g)) & 0xffu);
#pragma unroll
        for (int w = 0; w < TT; w++) {
            const uint8_t* xt = xl + (kTile * w + col) * G::TSTR * 16 + 4 + 8 * g + 8 * b * Q8_0_BYTES;
            const float* dw = dxl + (w * G::NS + 8 * b) * kTile;
            const float* gw = gxl + (w * G::NS + 8 * b) * kTile;
            v4f_t accb = v4f_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int sb = 0; sb < 8; sb++) {
                const int c = sb >> 1, sh = (sb & 1) * 4;
                const long bw = pack2((Q[c][0] >> sh) & 0x0f0f0f0fu, (Q[c][1] >> sh) & 0x0f0f0f0fu);
                const uint32_t* xa = reinterpret_cast<const uint32_t*>(xt + sb * Q8_0_BYTES);
                const v4i_t cc = __builtin_amdgcn_mfma_i32_16x16x32_i8(pack2(xa[0], xa[1]), bw, zi, 0, 0, 0);
                const v4f_t dx = *reinterpret_cast<const v4f_t*>(dw + sb * kTile + 4 * g);
                const int scv = (int)(((sb < 4 ? sc03 : sc47) >> (8 * (sb & 3))) & 0xffu);
                // |S| < 2^17 and sc < 64: the 24-bit multiply is exact
                accb[0] = fmaf((float)__mul24(cc[0], scv), dx[0], accb[0]);
                accb[1] = fmaf((float)__mul24(cc[1], scv), dx[1], accb[1]);
                accb[2] = fmaf((float)__mul24(cc[2], scv), dx[2], accb[2]);
                accb[3] = fmaf((float)__mul24(cc[3], scv), dx[3], accb[3]);
            }
            v4f_t a2 = acc[w];
#pragma unroll
            for (int ii = 0; ii < 4; ii++) a2[ii] = fmaf(d, accb[ii], a2[ii]);
            v4f_t m2 = __builtin_amdgcn_mfma_f32_16x16x4f32(gw[g * kTile + col], am0, macc[w], 0, 0, 0);
            m2 = __builtin_amdgcn_mfma_f32_16x16x4f32(gw[(4 + g) * kTile + col], am1, m2, 0, 0, 0);
            acc[w] = lv ? a2 : acc[w];
            macc[w] = lv ? m2 : macc[w];
        }
        // the block's results are final here (not sunk towards the stores)
#pragma unroll
        for (int w = 0; w < TT; w++) {
#pragma unroll
            for (int ii = 0; ii < 4; ii++) asm volatile("" : "+v"(acc[w][ii]), "+v"(macc[w][ii]));
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if (o < rows) {
        float* dst = S == 1 ? Y : part + (size_t)ks * T * rows;
#pragma unroll
        for (int w = 0; w < TT; w++) {
            const v4f_t v = acc[w] - macc[w];
#pragma unroll
            for (int ii = 0; ii < 4; ii++) {
                const int tok = t0 + kTile * w + 4 * g + ii;
                if (tok < T) dst[(size_t)tok * rows + o] = v[ii];
            }
        }
    }
}

// Y[t][o] = sum over k = 0..S-1, in that order, of part[k][t][o]
__global__ __launch_bounds__(256) void k_gemm_splitk_sum(float* __restrict__ Y,
                                                         const float* __restrict__ part,
                                                         int n, int S) {
    const int i = (int)blockIdx.x * 256 + (int)threadIdx.x;
    if (i >= n) return;
    float sum = part[i];
    for (int k = 1; k < S; k++) sum += part[(size_t)k * n + i];
    Y[i] = sum;
}

// The same sums four outputs per thread (n % 4 == 0, Y and part 16-byte
// aligned): a quarter of the load instructions; every partial's loads are
// issued before the first add.
template <int S>
__global__ __launch_bounds__(256) void k_gemm_splitk_sum4(float4* __restrict__ Y,
                                                          const float4* __restrict__ part,
                                                          int n4) {
    const int i = (int)blockIdx.x * 256 + (int)threadIdx.x;
    if (i >= n4) return;
    float4 v[S];
#pragma unroll
    for (int k = 0; k < S; k++) v[k] = part[(size_t)k * n4 + i];
    float4 sum = v[0];
#pragma unroll
    for (int k = 1; k < S; k++) {
        sum.x += v[k].x;
        sum.y += v[k].y;
        sum.z += v[k].z;
        sum.w += v[k].w;
    }
    Y[i] = sum;
}

// ---------------------------------------------------------------------------
// Q4_K x Q8_0 for wide token tiles on the fp16 matrix cores, the same sums
// with the 6-bit sub-block scale folded into the weight operand:
//   A (weight rows) = q*sc as fp16, B (tokens) = the int8 values as fp16.
// q <= 15 and sc <= 63 make q*sc <= 945, and |x| <= 128, so every operand,
// product and partial sum of one 32-value sub-block is an integer below 2^24:
// v_mfma_f32_16x16x32_f16 returns sc*S exactly, the int8 kernel's
// __mul24(S, sc).  The scaling that follows (dx per sub-block, d per block,
// the min term on the fp32 matrix cores) is the int8 kernel's, operation for
// operation; the 8 sub-blocks of a block are summed in order (the int8 kernel
// splits them over waves when a workgroup has fewer tiles than waves, which
// changes fp32 rounding only).  What changes is the work
// per tile: one FMA per result instead of a multiply, a conversion and an FMA,
// and the weight operand is built once per row tile for the wave's token tiles
// (v_perm_b32 makes fp16 1024+q, one v_pk_fma_f16 gives (1024+q)*sc - 1024*sc).
// With weights as A and tokens as B, a result lane holds rows 4g..4g+3 of one
// token: dx is one value per lane and sub-block.
//
// Workgroup: RT waves, wave w owns weight rows 16w..16w+15 and all 16*TTW
// tokens (TTW token tiles) of the workgroup; one Q4_K block per ring stage.
typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Rows o..o+3 of one token's output row y (o % 4 == 0): y[o+i] = v[i], or
// y[o+i] + v[i] when accumulating; one 16-byte access when vec (rows % 4 == 0
// and y 16-byte aligned), else per row below `rows`.
__device__ __forceinline__ void store_rows4(float* __restrict__ y, int o, int rows, v4f_t v,
                                            int accumulate, bool vec) {
    if (vec) {
        if (o >= rows) return;
        float4* p = reinterpret_cast<float4*>(y + o);
        float4 r = make_float4(v[0], v[1], v[2], v[3]);
        if (accumulate) {
            const float4 a = *p;
            r = make_float4(a.x + v[0], a.y + v[1], a.z + v[2], a.w + v[3]);
        }
        *p = r;
        return;
    }
#pragma unroll
    for (int ii = 0; ii < 4; ii++)
        if (o + ii < rows) y[o + ii] = accumulate ? y[o + ii] + v[ii] : v[ii];
}

// Activation re-layout for the fp16 kernel (TW = 16*TTW tokens per workgroup,
// Tp % TW == 0; slots past T zero):
//   xh [kb][g][t][8]                   fp16 copies of values 8g..8g+7 of record kb
//   dxt[kb][t/TW][t%16][(t/16)%TTW]    d     (one read: a lane's TTW token tiles)
//   gxt                                d * (sum of the 32 int8), same layout
template <int TTW>
__global__ __launch_bounds__(256) void k_gemm_prep16(const uint8_t* __restrict__ XQ8, int T,
                                                     int Tp, int nkb, uint8_t* __restrict__ xh,
                                                     float* __restrict__ dxt,
                                                     float* __restrict__ gxt) {
    constexpr int TW = 16 * TTW;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;  // kb * Tp + t
    if (i >= (long)nkb * Tp) return;
    const int t = (int)(i % Tp), kb = (int)(i / Tp);
    uint32_t w[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    float d = 0.f;
    int sum = 0;
    if (t < T) {
        const uint8_t* p = XQ8 + ((size_t)t * nkb + kb) * Q8_0_BYTES;
        d = __uint_as_float(ld4(p));
#pragma unroll
        for (int k = 0; k < 8; k++) {
            w[k] = ld4(p + 4 + 4 * k);
            sum = dot4((int)w[k], 0x01010101, sum);
        }
    }
#pragma unroll
    for (int g = 0; g < 4; g++) {
        v8h_t v;
#pragma unroll
        for (int e = 0; e < 8; e++)
            v[e] = (_Float16)(float)(int8_t)(w[2 * g + e / 4] >> (8 * (e % 4)));
        *reinterpret_cast<v8h_t*>(xh + (((size_t)kb * 4 + g) * Tp + t) * 16) = v;
    }
    const size_t q = (((size_t)kb * (Tp / TW) + t / TW) * 16 + (t & 15)) * TTW + ((t >> 4) % TTW);
    dxt[q] = d;
    gxt[q] = d * (float)sum;
}

// One stage: [RW rows][144 B] weights | xh [8][4][TW][16 B] | dxt [8][16][TTW] | gxt [8][16][TTW]
template <int RT, int TTW, int S>
struct Stage16 {
    static constexpr int NW = RT, RW = kTile * RT, TW = kTile * TTW;
    static constexpr int WB = RW * Q4K_BYTES;
    static constexpr int XB = 8 * 4 * TW * 16;
    static constexpr int DB = 8 * TW * 4;
    static constexpr int BYTES = WB + XB + 2 * DB;
    static constexpr int PIECES = (BYTES + 1023) / 1024;
    static constexpr int ALLOC = PIECES * 1024;
    static constexpr int PMAX = (PIECES + NW - 1) / NW;
    static constexpr int PMIN = PIECES / NW;
    static_assert(WB % 16 == 0 && XB % 1024 == 0 && DB % 128 == 0, "piece alignment");
    static_assert(S * ALLOC <= 160 * 1024, "LDS");
};

// N consecutive floats from LDS (N = 2 or 4: one 8- or 16-byte read)
template <int N>
__device__ __forceinline__ void lds_floats(const float* p, float (&out)[N]) {
    if constexpr (N == 4) {
        const float4 v = *reinterpret_cast<const float4*>(p);
        out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
    } else {
        static_assert(N == 2, "2 or 4 token tiles");
        const float2 v = *reinterpret_cast<const float2*>(p);
        out[0] = v.x; out[1] = v.y;
    }
}

// fp16 pair (1024 + n0, 1024 + n1) from two nibbles in bytes of u (v_perm_b32),
// then (1024 + n)*sc - 1024*sc = n*sc, exact (one rounding of an exact value)
__device__ __forceinline__ uint32_t nib_times_sc(uint32_t u, uint32_t sel, h2_t sc2, h2_t off2) {
    const uint32_t bits = __builtin_amdgcn_perm(0x64646464u, u, sel);
    const h2_t r = __builtin_elementwise_fma(__builtin_bit_cast(h2_t, bits), sc2, off2);
    return __builtin_bit_cast(uint32_t, r);
}

template <int RT, int TTW, int S>
__device__ __forceinline__ void gemm16_step(
    const uint8_t* __restrict__ cur, uint8_t* __restrict__ nxt, bool do_copy, int bnext, int i,
    int nb, const uint8_t* const (&src)[Stage16<RT, TTW, S>::PMAX],
    const uint32_t (&step)[Stage16<RT, TTW, S>::PMAX], int wave, int lane, int col, int g,
    v4f_t (&acc)[TTW], v4f_t (&macc)[TTW]) {
    using G = Stage16<RT, TTW, S>;
    constexpr int NW = G::NW, TW = G::TW;
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
    wait_later<G::PMIN, S - 1>(min(S - 1, nb - 1 - i));
    __builtin_amdgcn_s_barrier();

    const uint8_t* wl = cur + (kTile * wave + col) * Q4K_BYTES;  // this lane's A row
    const uint8_t* xl = cur + G::WB;
    const float* dl = reinterpret_cast<const float*>(cur + G::WB + G::XB);
    const float* gl = dl + 8 * TW;
    const uint4 h = *reinterpret_cast<const uint4*>(wl);
    const float dmin = h2f(h.x >> 16);
    const uint32_t sc03 = h.y & 0x3f3f3f3fu;
    const uint32_t sc47 = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
    long qv[4];
#pragma unroll
    for (int p = 0; p < 4; p++) qv[p] = *reinterpret_cast<const long*>(wl + 16 + 32 * p + 8 * g);

    const v4f_t zero = {0.f, 0.f, 0.f, 0.f};
    v4f_t accb[TTW];
#pragma unroll
    for (int j = 0; j < TTW; j++) accb[j] = zero;
#pragma unroll
    for (int s = 0; s < 8; s++) {
        // fp16 pair (1024 + sc, 1024 + sc) from byte s & 3 of the scale word
        // (v_perm_b32), minus 1024: sc exactly, and -1024*sc (<= 64512) exactly
        const uint32_t k = (uint32_t)(s & 3);
        const uint32_t scb = __builtin_amdgcn_perm(0x64646464u, s < 4 ? sc03 : sc47,
                                                   0x04000400u | (k << 16) | k);
        const h2_t m1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
        const h2_t sc2 = __builtin_bit_cast(h2_t, scb) + m1024;
        const h2_t off2 = sc2 * m1024;
        const int sh = 4 * (s & 1);
        const uint32_t u0 = ((uint32_t)qv[s >> 1] >> sh) & 0x0f0f0f0fu;
        const uint32_t u1 = ((uint32_t)((uint64_t)qv[s >> 1] >> 32) >> sh) & 0x0f0f0f0fu;
        const u32x4_t aw = {nib_times_sc(u0, 0x04010400u, sc2, off2),
                            nib_times_sc(u0, 0x04030402u, sc2, off2),
                            nib_times_sc(u1, 0x04010400u, sc2, off2),
                            nib_times_sc(u1, 0x04030402u, sc2, off2)};
        const v8h_t a = __builtin_bit_cast(v8h_t, aw);
        float dxs[TTW];
        lds_floats<TTW>(dl + (s * 16 + col) * TTW, dxs);
        v4f_t c[TTW];
#pragma unroll
        for (int j = 0; j < TTW; j++) {
            const v8h_t b =
                *reinterpret_cast<const v8h_t*>(xl + ((s * 4 + g) * TW + 16 * j + col) * 16);
            c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, zero, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < TTW; j++) {
#pragma unroll
            for (int ii = 0; ii < 4; ii++) accb[j][ii] = fmaf(c[j][ii], dxs[j], accb[j][ii]);
        }
    }
    // d of the result rows 4g..4g+3
    float dout[4];
#pragma unroll
    for (int ii = 0; ii < 4; ii++)
        dout[ii] = h2f(*reinterpret_cast<const uint16_t*>(cur + (kTile * wave + 4 * g + ii) *
                                                          Q4K_BYTES));
#pragma unroll
    for (int j = 0; j < TTW; j++) {
#pragma unroll
        for (int ii = 0; ii < 4; ii++) acc[j][ii] = fmaf(dout[ii], accb[j][ii], acc[j][ii]);
    }
    // min term: A = dmin*m (row col, sub-blocks g and 4+g), B = d*sum (tokens)
    const uint32_t m03 = h.z & 0x3f3f3f3fu;
    const uint32_t m47 = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
    const float am0 = dmin * (float)((m03 >> (8 * g)) & 0xffu);
    const float am1 = dmin * (float)((m47 >> (8 * g)) & 0xffu);
    float g0[TTW], g1[TTW];
    lds_floats<TTW>(gl + (g * 16 + col) * TTW, g0);
    lds_floats<TTW>(gl + ((4 + g) * 16 + col) * TTW, g1);
#pragma unroll
    for (int j = 0; j < TTW; j++) {
        macc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(am0, g0[j], macc[j], 0, 0, 0);
        macc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(am1, g1[j], macc[j], 0, 0, 0);
    }
    // stage free for chunk i + S
    __builtin_amdgcn_s_barrier();
}

// grid = 8 * ceil(nrt / 8) * (Tp / TW) workgroups, XCD-aware: workgroup L runs
// on XCD L % 8 (round-robin dispatch), and every token group of a row tile
// runs on one XCD, so the tile's weights are fetched into that XCD's L2 once.
// SW: the matrix is ffn_gate|ffn_up interleaved by blocks of 8 rows (8 gate
// rows, then the same 8 up rows), so a workgroup's 128 rows are 64
// consecutive SwiGLU pairs: the epilogue writes h = swiglu(gate, up) as the
// Q8_0 blocks of [T][rows / 2] (hq8) and, when hf is set, as fp32 rows,
// instead of Y; the arithmetic of k_swiglu_gu.  With hxh set it also writes
// those blocks' re-layout for the down projection's fp16 GEMM (hxh, hdx2,
// hgx2, hdx4 as k_rmsnorm_prep's, for the Tp tokens of the grid; tokens T..Tp-1
// zero).
template <int RT, int TTW, int S, bool SW = false>
__global__ __launch_bounds__(RT * 64) void k_gemm_f16_q4k(
    float* __restrict__ Y, const uint8_t* __restrict__ W, const uint8_t* __restrict__ xh,
    const float* __restrict__ dxt, const float* __restrict__ gxt, int rows, int nb,
    long row_bytes, int T, int Tp, int nrt, int accumulate, uint8_t* __restrict__ hq8 = nullptr,
    float* __restrict__ hf = nullptr, uint8_t* __restrict__ hxh = nullptr,
    float* __restrict__ hdx2 = nullptr, float* __restrict__ hgx2 = nullptr,
    float* __restrict__ hdx4 = nullptr) {
    using G = Stage16<RT, TTW, S>;
    constexpr int NW = G::NW, RW = G::RW, TW = G::TW;
    __shared__ __attribute__((aligned(16))) uint8_t smem[S * G::ALLOC];
    const int ntg = Tp / TW;
    const int L = blockIdx.x, xcd = L & 7, k = L >> 3;
    const int rt = (k / ntg) * 8 + xcd, ty = k % ntg;
    if (rt >= nrt) return;  // the whole workgroup, before any barrier
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int col = lane & 15, g = lane >> 4;
    const int row_base = rt * RW, tok_base = ty * TW;

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
            const int x = o - G::WB, s = x / (4 * TW * 16), gg = (x / (TW * 16)) & 3,
                      t = (x % (TW * 16)) / 16;
            src[j] = xh + (((size_t)s * 4 + gg) * Tp + tok_base + t) * 16;
            step[j] = 8u * 4u * (uint32_t)Tp * 16u;
        } else {
            const int y = o - G::WB - G::XB, which = y / G::DB, z = y - which * G::DB;
            const float* base = which == 0 ? dxt : gxt;
            src[j] = reinterpret_cast<const uint8_t*>(base) +
                     ((size_t)(z / (TW * 4)) * (Tp / TW) + tok_base / TW) * (TW * 4) +
                     (z % (TW * 4));
            step[j] = 8u * (uint32_t)Tp * 4u;
        }
    }
    v4f_t acc[TTW], macc[TTW];
#pragma unroll
    for (int j = 0; j < TTW; j++) {
        acc[j] = v4f_t{0.f, 0.f, 0.f, 0.f};
        macc[j] = v4f_t{0.f, 0.f, 0.f, 0.f};
    }
    for (int i = 1 - S; i < nb; i++) {
        const int inext = i + S - 1;
        gemm16_step<RT, TTW, S>(smem + ((i + S) % S) * G::ALLOC, smem + (inext % S) * G::ALLOC,
                                inext < nb, inext, i, nb, src, step, wave, lane, col, g, acc,
                                macc);
    }
    if constexpr (SW) {
        static_assert(RT == 8, "64 SwiGLU pairs per workgroup: two Q8_0 blocks");
        // lane (col, g < 2) holds gate rows 4g..4g+3 of the wave's 8 pairs, lane
        // (col, g + 2) the matching up rows; the ring's LDS is free (the last
        // step ended with a barrier): h[token][64] of this workgroup
        float* hs = reinterpret_cast<float*>(smem);
#pragma unroll
        for (int j = 0; j < TTW; j++) {
            const v4f_t v = acc[j] - macc[j];
#pragma unroll
            for (int ii = 0; ii < 4; ii++) {
                const float up = __shfl_xor(v[ii], 32, 64);
                if (g < 2) hs[(16 * j + col) * 64 + 8 * wave + 4 * g + ii] = swiglu1(v[ii], up);
            }
        }
        __syncthreads();
        // 8 lanes per Q8_0 block (4 values each), as k_swiglu_gu: 2 blocks x TW tokens
        const int nh = rows / 2;
        for (int q = threadIdx.x; q < TW * 16; q += RT * 64) {
            const int tl = q >> 4, half = (q >> 3) & 1, sub = q & 7, tok = tok_base + tl;
            const float4 o = *reinterpret_cast<const float4*>(hs + tl * 64 + 32 * half + 4 * sub);
            // the 8 lanes of a block share the token
            const int kb = 2 * rt + half;  // block of h's row
            float d = 0.f;
            uint32_t p = 0u;
            if (tok < T) {
                const size_t e = (size_t)tok * nh + 64 * rt + 32 * half + 4 * sub;
                if (hf) *reinterpret_cast<float4*>(hf + e) = o;
                p = q8_quant4(o, d);  // q8_block_store's block
                uint8_t* blk = hq8 + (e >> 5) * Q8_0_BYTES;
                *reinterpret_cast<uint32_t*>(blk + 4 + 4 * sub) = p;
                if (sub == 0) *reinterpret_cast<float*>(blk) = d;
            }
            if (hxh) {  // k_gemm_prep16's re-layout of the block (zeros past T)
                _Float16 hv[4];
#pragma unroll
                for (int e = 0; e < 4; e++) hv[e] = (_Float16)(float)(int8_t)(p >> (8 * e));
                *reinterpret_cast<uint2*>(hxh + (((size_t)kb * 4 + (sub >> 1)) * Tp + tok) * 16 +
                                          (sub & 1) * 8) = *reinterpret_cast<const uint2*>(hv);
                int sum = dot4((int)p, 0x01010101, 0);
                sum += __shfl_xor(sum, 1, 8);
                sum += __shfl_xor(sum, 2, 8);
                sum += __shfl_xor(sum, 4, 8);
                if (sub == 0) {
                    const size_t i2 = (((size_t)kb * (Tp / 32) + tok / 32) * 16 + (tok & 15)) * 2 + ((tok >> 4) & 1);
                    const size_t i4 = (((size_t)kb * (Tp / 64) + tok / 64) * 16 + (tok & 15)) * 4 + ((tok >> 4) & 3);
                    hdx2[i2] = d;
                    hgx2[i2] = d * (float)sum;
                    hdx4[i4] = d;
                }
            }
        }
        return;
    }
    // a lane's 4 consecutive rows of one token as one 16-byte access where
    // rows % 4 == 0 (the same adds)
    const bool vec = (rows & 3) == 0 && ((uintptr_t)Y & 15) == 0;
#pragma unroll
    for (int j = 0; j < TTW; j++) {
        const v4f_t v = acc[j] - macc[j];
        const int tok = tok_base + 16 * j + col;
        if (tok < T) store_rows4(Y + (size_t)tok * rows, row_base + kTile * wave + 4 * g, rows,
                                 v, accumulate, vec);
    }
}

template <int RT, int TTW, int S>
void launch16_cfg(float* Y, const uint8_t* W, const uint8_t* XQ8, uint8_t* scratch, int rows,
                  int nb, long row_bytes, int T, hipStream_t st, int accumulate) {
    constexpr int TW = kTile * TTW;
    const int Tp = (T + TW - 1) / TW * TW, nkb = nb * 8;
    auto* xh = scratch;
    auto* dxt = reinterpret_cast<float*>(xh + (size_t)nkb * Tp * 64);
    auto* gxt = dxt + (size_t)nkb * Tp;
    const long n = (long)nkb * Tp;
    hipLaunchKernelGGL(k_gemm_prep16<TTW>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       XQ8, T, Tp, nkb, xh, dxt, gxt);
    const int nrt = (rows + kTile * RT - 1) / (kTile * RT);
    const unsigned grid = (unsigned)((nrt + 7) / 8 * 8 * (Tp / TW));
    hipLaunchKernelGGL((k_gemm_f16_q4k<RT, TTW, S>), dim3(grid), dim3(RT * 64), 0, st, Y, W, xh,
                       dxt, gxt, rows, nb, row_bytes, T, Tp, nrt, accumulate);
}

// ---------------------------------------------------------------------------
// Q6_K x Q8_0 on the matrix cores.  Per (token t, row o):
//   Y = sum_b d * sum_s sc_s * dx_s * sum_k (q_k - 32) x_k
// over the 16-weight sub-blocks s (the per-token dot of
// gemv_q6k_q8_avx2_range, gemv_q6k_q8_avx2.cpp:104-205, which gemm_wt_q8 runs
// per token for Q6_K weights, llama_model.cpp:860-873).
//   * B = the signed 6-bit weights q - 32 in [-32, 31] as int8: low nibble from
//     ql, high nibble (h - 2) mod 16 from the two qh bits h, which is exact;
//   * one Q8_0 block (32 k) covers two sub-blocks with their own int8 scales,
//     so it takes two v_mfma_i32_16x16x32_i8 whose B has the other
//     sub-block's k-groups zeroed; sc is applied by 24-bit integer
//     multiply-adds (exact in int32), dx by an fp32 FMA, d once per block.
// Stage layout: KS super-blocks, each RW rows x 224-byte slots holding the
// 16-byte-aligned span that covers the row's 210-byte block (blocks are 2-byte
// aligned), then the KS super-blocks' int8 activations and dx (as for Q4_K).
// A span starts up to 14 bytes before its block and ends up to 14 bytes after
// it; the launcher takes this kernel only when the matrix's last block ends on
// a 16-byte boundary, so every span lies in [W rounded down to 16 bytes, end
// of the last block).  The spans are copied by buffer loads whose resource is
// exactly that range.
// Waves: KS groups (one super-block of the stage each) x RT row tiles x TS
// token splits; the KS partial sums are added in a fixed order through LDS.
// ---------------------------------------------------------------------------
template <int RT, int TT, int KS, int TS, int S>
struct Stage6 {
    static constexpr int RW = kTile * RT, TW = kTile * TT;
    static constexpr int NW = KS * RT * TS;
    // a row's span is 224 bytes (14 pieces of 16); the slot is 240 bytes so
    // that the 16 rows a wave reads sit 60 banks apart
    static constexpr int SPAN = 224, SLOT = 240;
    static constexpr int WSB = RW * SLOT;     // weights of one super-block
    static constexpr int XSB = 8 * TW * 32;   // int8 activations of one super-block
    static constexpr int DSB = 8 * TW * 4;    // dx of one super-block
    static constexpr int WB = KS * WSB, XB = KS * XSB, DB = KS * DSB;
    static constexpr int BYTES = WB + XB + DB;
    static constexpr int PIECES = (BYTES + 1023) / 1024;
    static constexpr int ALLOC = PIECES * 1024;
    static constexpr int PMAX = (PIECES + NW - 1) / NW;
    static constexpr int PMIN = PIECES / NW;
    static constexpr int WP = WB / 1024;  // pieces 0..WP-1 hold weights
    static constexpr int WT = TT / TS;    // token tiles per wave
    static_assert(TT % TS == 0, "token split");
    static_assert(WB % 1024 == 0 && XSB % 16 == 0 && DSB % 16 == 0, "piece alignment");
    static_assert(NW <= 16, "workgroup size");
};

// N dwords of LDS bytes at p0 + off, p0 4-byte aligned, off any byte offset
// (the address stays an LDS pointer: aligned ds_read_b32 + v_alignbyte)
template <int N>
__device__ __forceinline__ void lds_bytes(const uint8_t* p0, uint32_t off, uint32_t (&out)[N]) {
    const uint32_t* base = reinterpret_cast<const uint32_t*>(p0 + (off & ~3u));
    const uint32_t sh = off & 3u;
    uint32_t w[N + 1];
#pragma unroll
    for (int k = 0; k <= N; k++) w[k] = base[k];
#pragma unroll
    for (int k = 0; k < N; k++) out[k] = __builtin_amdgcn_alignbyte(w[k + 1], w[k], sh);
}

// Per copy piece of this lane: weights — base = the row's offset in the
// buffer resource, aux = the lane's offset in the slot; activations — base =
// the address for super-block 0, aux = bytes per super-block.  ks = the
// piece's super-block within the stage.
template <int RT, int TT, int KS, int TS, int S>
struct Plan6 {
    uint64_t base[Stage6<RT, TT, KS, TS, S>::PMAX];
    uint32_t aux[Stage6<RT, TT, KS, TS, S>::PMAX];
    uint32_t ks[Stage6<RT, TT, KS, TS, S>::PMAX];
};

template <int RT, int TT, int KS, int TS, int S>
__device__ __forceinline__ void gemm6_step(
    const uint8_t* __restrict__ cur, uint8_t* __restrict__ nxt, bool do_copy, int snext, int i,
    int nst, int nb, const Plan6<RT, TT, KS, TS, S>& pl, __amdgpu_buffer_rsrc_t wrsrc, int wave, int col, int g, int ksw, int rt, int tt0,
    uint32_t wlo, v4f_t (&acc)[Stage6<RT, TT, KS, TS, S>::WT]) {
    using G = Stage6<RT, TT, KS, TS, S>;
    constexpr int TW = G::TW, NW = G::NW;
    if (do_copy) {
#pragma unroll
        for (int j = 0; j < G::PMAX; j++) {
            const int piece = wave + NW * j;
            // super-block of this piece (past the end: the last one again, unused)
            const uint32_t b = min((uint32_t)(snext * KS) + pl.ks[j], (uint32_t)(nb - 1));
            if (piece < G::WP) {
                // the aligned span of the row's block b; this lane's 16 bytes sit
                // aux[j] bytes into the slot
                const uint32_t o =
                    (((uint32_t)pl.base[j] + b * (uint32_t)Q6K_BYTES) & ~15u) + pl.aux[j];
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wrsrc, (lmem_t*)(nxt + piece * 1024), 16,
                                                         o, 0, 0, 0);
            } else if (piece < G::PIECES) {
                const uint8_t* a =
                    reinterpret_cast<const uint8_t*>(pl.base[j]) + (size_t)b * pl.aux[j];
                __builtin_amdgcn_global_load_lds((gmem_t*)a, (lmem_t*)(nxt + piece * 1024), 16,
                                                 0, 0);
            }
        }
    }
    if (i < 0) return;
    const int later = min(S - 1, nst - 1 - i);
    wait_later<G::PMIN, S - 1>(later);
    __builtin_amdgcn_s_barrier();

    const int b = i * KS + ksw;  // this wave's super-block
    if (b < nb) {
        // this lane's weight row: its block starts (wlo + 2b) & 15 bytes into the slot
        const uint8_t* wl = cur + ksw * G::WSB + (kTile * rt + col) * G::SLOT;
        const uint32_t wo = (wlo + 2u * (uint32_t)b) & 15u;
        const uint8_t* xl = cur + G::WB + ksw * G::XSB;
        const float* dl = reinterpret_cast<const float*>(cur + G::WB + G::XB + ksw * G::DSB);
        uint32_t ql[2][2][2], qh[2][2], sc[4], dw[1];
#pragma unroll
        for (int n = 0; n < 2; n++) {
#pragma unroll
            for (int h = 0; h < 2; h++) lds_bytes<2>(wl, wo + 64 * n + 32 * h + 8 * g, ql[n][h]);
            lds_bytes<2>(wl, wo + 128 + 32 * n + 8 * g, qh[n]);
        }
        lds_bytes<4>(wl, wo + 192, sc);
        lds_bytes<1>(wl, wo + 208, dw);
        const float d = h2f(dw[0] & 0xffffu);
        const v4i_t zi = {0, 0, 0, 0};
        // k-groups 0,1 are the block's first sub-block, k-groups 2,3 its second
        const uint64_t m1 = g < 2 ? ~0ull : 0ull;
        v4f_t accb[G::WT];
#pragma unroll
        for (int w = 0; w < G::WT; w++) accb[w] = v4f_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 8; kb++) {
            const int n = kb >> 2, q = kb & 3, h = q & 1, nib = q >> 1;
            uint32_t v[2];
#pragma unroll
            for (int x = 0; x < 2; x++) {
                // bytes q - 32: low nibble | ((hi2 + 14) mod 16) << 4
                const uint32_t lo = (ql[n][h][x] >> (4 * nib)) & 0x0f0f0f0fu;
                const uint32_t hi = (((qh[n][x] >> (2 * q)) & 0x03030303u) + 0x0e0e0e0eu) &
                                    0x0f0f0f0fu;
                v[x] = lo | (hi << 4);
            }
            const uint64_t bw = ((uint64_t)v[1] << 32) | v[0];
            const long b1 = (long)(bw & m1), b2 = (long)(bw & ~m1);
            const int s1 = (int)(int8_t)(sc[kb >> 1] >> (16 * (kb & 1)));
            const int s2 = (int)(int8_t)(sc[kb >> 1] >> (16 * (kb & 1) + 8));
#pragma unroll
            for (int w = 0; w < G::WT; w++) {
                const int tok = kTile * (tt0 + w);
                // (a scalar 64-bit read: its LDS access keeps the noalias scope
                // that lets the copies into the other stage buffers stay in flight)
                const long a = *reinterpret_cast<const long*>(
                    xl + (kb * TW + tok + col) * 32 + 8 * (g ^ (2 * ((col >> 3) & 1))));
                const float4 dx = *reinterpret_cast<const float4*>(dl + kb * TW + tok + 4 * g);
                const v4i_t c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b1, zi, 0, 0, 0);
                const v4i_t c2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b2, zi, 0, 0, 0);
                // |c| <= 16 * 128 * 32 and |sc| <= 128: the 24-bit products are exact
                accb[w][0] = fmaf((float)(__mul24(c2[0], s2) + __mul24(c1[0], s1)), dx.x, accb[w][0]);
                accb[w][1] = fmaf((float)(__mul24(c2[1], s2) + __mul24(c1[1], s1)), dx.y, accb[w][1]);
                accb[w][2] = fmaf((float)(__mul24(c2[2], s2) + __mul24(c1[2], s1)), dx.z, accb[w][2]);
                accb[w][3] = fmaf((float)(__mul24(c2[3], s2) + __mul24(c1[3], s1)), dx.w, accb[w][3]);
            }
        }
#pragma unroll
        for (int w = 0; w < G::WT; w++)
#pragma unroll
            for (int ii = 0; ii < 4; ii++) acc[w][ii] = fmaf(d, accb[w][ii], acc[w][ii]);
    }
    __builtin_amdgcn_s_barrier();
}

// Workgroup = NW waves on a (16*RT rows) x (16*TT tokens) tile; stage i holds
// super-blocks i*KS .. i*KS + KS - 1.
template <int RT, int TT, int KS, int TS, int S>
__global__ __launch_bounds__(KS * RT * TS * 64) void k_gemm_mfma_q6k(
    float* __restrict__ Y, const uint8_t* __restrict__ W, const uint8_t* __restrict__ xs,
    const float* __restrict__ dxs, int rows, int nb, long row_bytes, int T, int Tp, int accumulate) {
    using G = Stage6<RT, TT, KS, TS, S>;
    constexpr int RW = G::RW, TW = G::TW, NW = G::NW;
    __shared__ __attribute__((aligned(16))) uint8_t smem[S * G::ALLOC];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, g = lane >> 4;
    const int row_base = blockIdx.x * RW;
    const int tok_base = blockIdx.y * TW;

    // weights through a buffer resource from W rounded down to 16 bytes to the
    // end of the last block (the host checks that this is under 2 GiB)
    const uint32_t w0 = (uint32_t)(reinterpret_cast<uintptr_t>(W) & 15);
    const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(W - w0), 0,
        (int)(w0 + (uint32_t)(rows - 1) * (uint32_t)row_bytes + (uint32_t)nb * Q6K_BYTES),
        0x00020000);
    // activations: xs [8b + k][Tp][32] and dxs [8b + k][Tp] for super-block b
    Plan6<RT, TT, KS, TS, S> pl;
#pragma unroll
    for (int j = 0; j < G::PMAX; j++) {
        int o = (wave + NW * j) * 1024 + lane * 16;
        if (o >= G::BYTES) o = G::WB;  // tail of the last piece: a harmless duplicate
        if (o < G::WB) {
            const int ks = o / G::WSB, y = o - ks * G::WSB, r = y / G::SLOT;
            pl.ks[j] = (uint32_t)ks;
            pl.base[j] = w0 + (uint32_t)min(row_base + r, rows - 1) * (uint32_t)row_bytes;
            const int a = y - r * G::SLOT;
            pl.aux[j] = (uint32_t)(a < G::SPAN ? a : 0);  // slot padding: a duplicate
        } else if (o < G::WB + G::XB) {
            const int x = o - G::WB, ks = x / G::XSB, y = x - ks * G::XSB, k = y / (TW * 32);
            // token t's two 16-byte halves are swapped in LDS when bit 3 of t is
            // set, so the 8-byte reads of 32 lanes (16 tokens x 2 k-groups) hit
            // distinct banks
            const int r = y - k * TW * 32, t = r >> 5, hb = ((r >> 4) & 1) ^ ((t >> 3) & 1);
            pl.ks[j] = (uint32_t)ks;
            pl.base[j] = reinterpret_cast<uint64_t>(xs + ((size_t)k * Tp + tok_base) * 32 +
                                                    t * 32 + hb * 16);
            pl.aux[j] = 8u * (uint32_t)Tp * 32u;
        } else {
            const int x = o - G::WB - G::XB, ks = x / G::DSB, y = x - ks * G::DSB,
                      k = y / (TW * 4);
            pl.ks[j] = (uint32_t)ks;
            pl.base[j] = reinterpret_cast<uint64_t>(
                reinterpret_cast<const uint8_t*>(dxs + (size_t)k * Tp + tok_base) +
                (y - k * TW * 4));
            pl.aux[j] = 8u * (uint32_t)Tp * 4u;
        }
    }
    const int ksw = wave / (RT * TS), rr = wave % (RT * TS);
    const int rt = rr % RT, tt0 = (rr / RT) * G::WT;
    const uint32_t wlo =
        (w0 + (uint32_t)min(row_base + kTile * rt + col, rows - 1) * (uint32_t)row_bytes) & 15u;
    v4f_t acc[G::WT];
#pragma unroll
    for (int w = 0; w < G::WT; w++) acc[w] = v4f_t{0.f, 0.f, 0.f, 0.f};
    const int nst = (nb + KS - 1) / KS;
    for (int i = 1 - S; i < nst; i++) {
        const int inext = i + S - 1;
        gemm6_step<RT, TT, KS, TS, S>(smem + ((i + S) % S) * G::ALLOC,
                                      smem + (inext % S) * G::ALLOC, inext < nst, inext, i, nst,
                                      nb, pl, wrsrc, wave, col, g, ksw, rt, tt0, wlo, acc);
    }
    // sum the KS partial tiles in a fixed order (group 0 + 1 + ... + KS-1)
    if constexpr (KS > 1) {
        float* red = reinterpret_cast<float*>(smem);
        static_assert((KS - 1) * RT * TT * 64 * 16 <= S * G::ALLOC, "reduction space");
        if (ksw > 0) {
#pragma unroll
            for (int w = 0; w < G::WT; w++)
                *reinterpret_cast<float4*>(
                    red + ((((ksw - 1) * RT + rt) * TT + tt0 + w) * 64 + lane) * 4) =
                    make_float4(acc[w][0], acc[w][1], acc[w][2], acc[w][3]);
        }
        __syncthreads();
        if (ksw > 0) return;
#pragma unroll
        for (int k = 1; k < KS; k++)
#pragma unroll
            for (int w = 0; w < G::WT; w++) {
                const float4 p = *reinterpret_cast<const float4*>(
                    red + ((((k - 1) * RT + rt) * TT + tt0 + w) * 64 + lane) * 4);
                acc[w][0] += p.x;
                acc[w][1] += p.y;
                acc[w][2] += p.z;
                acc[w][3] += p.w;
            }
    }
    const int o = row_base + kTile * rt + col;
    if (o < rows) {
#pragma unroll
        for (int w = 0; w < G::WT; w++) {
#pragma unroll
            for (int ii = 0; ii < 4; ii++) {
                const int tok = tok_base + kTile * (tt0 + w) + 4 * g + ii;
                if (tok < T) {
                    float* y = Y + (size_t)tok * rows + o;
                    *y = accumulate ? *y + acc[w][ii] : acc[w][ii];
                }
            }
        }
    }
}

template <int RT, int TT, int KS, int TS, int S>
void launch6_cfg(float* Y, const uint8_t* W, const uint8_t* xs, const float* dxs, int rows,
                 int nb, long row_bytes, int T, int Tp, hipStream_t st, int accumulate) {
    using G = Stage6<RT, TT, KS, TS, S>;
    const dim3 grid((unsigned)((rows + G::RW - 1) / G::RW), (unsigned)(Tp / G::TW));
    hipLaunchKernelGGL((k_gemm_mfma_q6k<RT, TT, KS, TS, S>), grid, dim3(G::NW * 64), 0, st, Y,
                       W, xs, dxs, rows, nb, row_bytes, T, Tp, accumulate);
}

// ---------------------------------------------------------------------------
// Q6_K x Q8_0 for wide token tiles on the fp16 matrix cores.  The per-16 scale
// goes into the weight operand as two exact fp16 codes per weight: with
// q - 32 = 16 hb + l (l = the low nibble in [0, 15], hb = the two high bits
// minus 2, in [-2, 1]),
//   c1 = sc * l       |c1| <= 128 * 15 = 1920: an fp16 integer
//   c2 = 16 * sc * hb |c2| <= 4096, a multiple of 16: an fp16 integer
// and B = the int8 activations as fp16 (exact).  Per Q8_0 block and token tile
// two v_mfma_f32_16x16x32_f16 (A = c1, then c2, one accumulator) return
// sum sc * (q - 32) * x over the block's two sub-blocks: integers below 2^24
// (|sc (q - 32) x| <= 128 * 32 * 127, 32 of them), so exact in fp32 and equal
// to the int8 kernel's sc1*S1 + sc2*S2.  Then one FMA with dx per result (the
// int8 kernel: two 24-bit multiplies, a conversion and the FMA) and d per
// super-block, as there.  Weights as A (rows), tokens as B, as in the fp16
// Q4_K kernel, whose activation re-layout (k_gemm_prep16) this one reads; d
// of the result rows 4g..4g+3 comes from the lanes holding those rows.
// Workgroup: RT waves, wave w owns rows 16w..16w+15 and the 16*TTW tokens;
// one super-block per ring stage: RW rows of 240-byte slots holding each
// row's 16-byte-aligned 224-byte span (as k_gemm_mfma_q6k), then the
// super-block's fp16 activations and dx (no min term for Q6_K).
// ---------------------------------------------------------------------------
template <int RT, int TTW, int S>
struct Stage6h {
    static constexpr int NW = RT, RW = kTile * RT, TW = kTile * TTW;
    static constexpr int SPAN = 224, SLOT = 240;
    static constexpr int WB = RW * SLOT;
    static constexpr int XB = 8 * 4 * TW * 16;
    static constexpr int DB = 8 * TW * 4;
    static constexpr int BYTES = WB + XB + DB;
    static constexpr int PIECES = (BYTES + 1023) / 1024;
    static constexpr int ALLOC = PIECES * 1024;
    static constexpr int PMAX = (PIECES + NW - 1) / NW;
    static constexpr int PMIN = PIECES / NW;
    static_assert(WB % 1024 == 0 && XB % 1024 == 0 && DB % 256 == 0, "piece alignment");
    static_assert(S * ALLOC <= 160 * 1024, "LDS");
};

// fp16 pairs of (byte - off) * scale for 4 bytes of u, exact where the
// products are fp16 integers: v_perm_b32 makes 1024 + byte, then one packed
// add and one packed multiply
__device__ __forceinline__ void bytes_scaled(uint32_t u, h2_t off2, h2_t sc2, uint32_t& lo,
                                             uint32_t& hi) {
    const h2_t a = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u));
    const h2_t b = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u));
    lo = __builtin_bit_cast(uint32_t, (a + off2) * sc2);
    hi = __builtin_bit_cast(uint32_t, (b + off2) * sc2);
}

template <int RT, int TTW, int S>
__device__ __forceinline__ void gemm6h_step(
    const uint8_t* __restrict__ cur, uint8_t* __restrict__ nxt, bool do_copy, int bnext, int i,
    int nb, const uint64_t (&base)[Stage6h<RT, TTW, S>::PMAX],
    const uint32_t (&aux)[Stage6h<RT, TTW, S>::PMAX], __amdgpu_buffer_rsrc_t wrsrc, int wave,
    int col, int g, uint32_t wlo, v4f_t (&acc)[TTW]) {
    using G = Stage6h<RT, TTW, S>;
    constexpr int NW = G::NW, TW = G::TW;
    if (do_copy) {
#pragma unroll
        for (int j = 0; j < G::PMAX; j++) {
            const int piece = wave + NW * j;
            if (piece * 1024 < G::WB) {
                // the aligned span of the row's block bnext; this lane's 16 bytes
                // sit aux[j] bytes into the slot
                const uint32_t o = (((uint32_t)base[j] + (uint32_t)bnext * (uint32_t)Q6K_BYTES) & ~15u) + aux[j];
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wrsrc, (lmem_t*)(nxt + piece * 1024), 16,
                                                         o, 0, 0, 0);
            } else if (piece < G::PIECES) {
                const uint8_t* a = reinterpret_cast<const uint8_t*>(base[j]) + (size_t)bnext * aux[j];
                __builtin_amdgcn_global_load_lds((gmem_t*)a, (lmem_t*)(nxt + piece * 1024), 16, 0,
                                                 0);
            }
        }
    }
    if (i < 0) return;
    wait_later<G::PMIN, S - 1>(min(S - 1, nb - 1 - i));
    __builtin_amdgcn_s_barrier();

    // this lane's row: its block starts (wlo + 2i) & 15 bytes into the slot
    const uint8_t* wl = cur + (kTile * wave + col) * G::SLOT;
    const uint32_t wo = (wlo + 2u * (uint32_t)i) & 15u;
    const uint8_t* xl = cur + G::WB;
    const float* dl = reinterpret_cast<const float*>(cur + G::WB + G::XB);
    uint32_t ql[2][2][2], qh[2][2], sc[4], dw[1];
#pragma unroll
    for (int n = 0; n < 2; n++) {
#pragma unroll
        for (int h = 0; h < 2; h++) lds_bytes<2>(wl, wo + 64 * n + 32 * h + 8 * g, ql[n][h]);
        lds_bytes<2>(wl, wo + 128 + 32 * n + 8 * g, qh[n]);
    }
    lds_bytes<4>(wl, wo + 192, sc);
    lds_bytes<1>(wl, wo + 208, dw);
    const v4f_t zero = {0.f, 0.f, 0.f, 0.f};
    v4f_t accb[TTW];
#pragma unroll
    for (int j = 0; j < TTW; j++) accb[j] = zero;
    const h2_t offl = {(_Float16)-1024.f, (_Float16)-1024.f};
    const h2_t offh = {(_Float16)-1026.f, (_Float16)-1026.f};
#pragma unroll
    for (int kb = 0; kb < 8; kb++) {
        const int n = kb >> 2, q = kb & 3, h = q & 1, nib = q >> 1;
        // k-group g: sub-block 2kb + (g >> 1), scale byte 2(kb & 1) + (g >> 1) of sc[kb >> 1]
        const int scv = (int)(int8_t)(sc[kb >> 1] >> (16 * (kb & 1) + 8 * (g >> 1)));
        const _Float16 s1 = (_Float16)(float)scv, s16 = (_Float16)(16.f * (float)scv);
        const h2_t sc1 = {s1, s1}, sc16 = {s16, s16};
        uint32_t c1[4], c2[4];
#pragma unroll
        for (int x = 0; x < 2; x++) {
            const uint32_t l = (ql[n][h][x] >> (4 * nib)) & 0x0f0f0f0fu;
            const uint32_t hb = (qh[n][x] >> (2 * q)) & 0x03030303u;
            bytes_scaled(l, offl, sc1, c1[2 * x], c1[2 * x + 1]);
            bytes_scaled(hb, offh, sc16, c2[2 * x], c2[2 * x + 1]);
        }
        const v8h_t a1 = __builtin_bit_cast(v8h_t, u32x4_t{c1[0], c1[1], c1[2], c1[3]});
        const v8h_t a2 = __builtin_bit_cast(v8h_t, u32x4_t{c2[0], c2[1], c2[2], c2[3]});
        float dxs[TTW];
        lds_floats<TTW>(dl + (kb * 16 + col) * TTW, dxs);
#pragma unroll
        for (int j = 0; j < TTW; j++) {
            const v8h_t b =
                *reinterpret_cast<const v8h_t*>(xl + ((kb * 4 + g) * TW + 16 * j + col) * 16);
            v4f_t c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b, zero, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, b, c, 0, 0, 0);
#pragma unroll
            for (int ii = 0; ii < 4; ii++) accb[j][ii] = fmaf(c[ii], dxs[j], accb[j][ii]);
        }
    }
    // d of the result rows 4g..4g+3: lane 4g + ii (g = 0 there) holds row 4g + ii
    const float down = h2f(dw[0] & 0xffffu);
    float dout[4];
#pragma unroll
    for (int ii = 0; ii < 4; ii++) dout[ii] = __shfl(down, 4 * g + ii, 64);
#pragma unroll
    for (int j = 0; j < TTW; j++)
#pragma unroll
        for (int ii = 0; ii < 4; ii++) acc[j][ii] = fmaf(dout[ii], accb[j][ii], acc[j][ii]);
    // stage free for chunk i + S
    __builtin_amdgcn_s_barrier();
}

// grid = 8 * ceil(nrt / 8) * (Tp / TW) workgroups, XCD-aware as k_gemm_f16_q4k
template <int RT, int TTW, int S>
__global__ __launch_bounds__(RT * 64) void k_gemm_f16_q6k(
    float* __restrict__ Y, const uint8_t* __restrict__ W, const uint8_t* __restrict__ xh,
    const float* __restrict__ dxt, int rows, int nb, long row_bytes, int T, int Tp, int nrt,
    int accumulate) {
    using G = Stage6h<RT, TTW, S>;
    constexpr int NW = G::NW, RW = G::RW, TW = G::TW;
    __shared__ __attribute__((aligned(16))) uint8_t smem[S * G::ALLOC];
    const int ntg = Tp / TW;
    const int L = blockIdx.x, xcd = L & 7, k = L >> 3;
    const int rt = (k / ntg) * 8 + xcd, ty = k % ntg;
    if (rt >= nrt) return;  // the whole workgroup, before any barrier
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int col = lane & 15, g = lane >> 4;
    const int row_base = rt * RW, tok_base = ty * TW;

    // weights through a buffer resource from W rounded down to 16 bytes to the
    // end of the last block (the host checks that this is under 2 GiB)
    const uint32_t w0 = (uint32_t)(reinterpret_cast<uintptr_t>(W) & 15);
    const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(W - w0), 0,
        (int)(w0 + (uint32_t)(rows - 1) * (uint32_t)row_bytes + (uint32_t)nb * Q6K_BYTES),
        0x00020000);
    // per piece of this lane: weights — base = the row's offset in the buffer
    // resource, aux = the lane's offset in the slot; activations — base = the
    // address for super-block 0, aux = bytes per super-block
    uint64_t base[G::PMAX];
    uint32_t aux[G::PMAX];
#pragma unroll
    for (int j = 0; j < G::PMAX; j++) {
        int o = (wave + NW * j) * 1024 + lane * 16;
        if (o >= G::BYTES) o = G::WB;  // tail of the last piece: a harmless duplicate
        if (o < G::WB) {
            const int r = o / G::SLOT, a = o - r * G::SLOT;
            base[j] = w0 + (uint32_t)min(row_base + r, rows - 1) * (uint32_t)row_bytes;
            aux[j] = (uint32_t)(a < G::SPAN ? a : 0);  // slot padding: a duplicate
        } else if (o < G::WB + G::XB) {
            const int x = o - G::WB, s = x / (4 * TW * 16), gg = (x / (TW * 16)) & 3,
                      t = (x % (TW * 16)) / 16;
            base[j] = reinterpret_cast<uint64_t>(xh + (((size_t)s * 4 + gg) * Tp + tok_base + t) * 16);
            aux[j] = 8u * 4u * (uint32_t)Tp * 16u;
        } else {
            const int z = o - G::WB - G::XB;
            base[j] = reinterpret_cast<uint64_t>(
                reinterpret_cast<const uint8_t*>(dxt) +
                ((size_t)(z / (TW * 4)) * (Tp / TW) + tok_base / TW) * (TW * 4) + (z % (TW * 4)));
            aux[j] = 8u * (uint32_t)Tp * 4u;
        }
    }
    const uint32_t wlo =
        (w0 + (uint32_t)min(row_base + kTile * wave + col, rows - 1) * (uint32_t)row_bytes) & 15u;
    v4f_t acc[TTW];
#pragma unroll
    for (int j = 0; j < TTW; j++) acc[j] = v4f_t{0.f, 0.f, 0.f, 0.f};
    for (int i = 1 - S; i < nb; i++) {
        const int inext = i + S - 1;
        gemm6h_step<RT, TTW, S>(smem + ((i + S) % S) * G::ALLOC, smem + (inext % S) * G::ALLOC,
                                inext < nb, inext, i, nb, base, aux, wrsrc, wave, col, g, wlo,
                                acc);
    }
    const bool vec = (rows & 3) == 0 && ((uintptr_t)Y & 15) == 0;
#pragma unroll
    for (int j = 0; j < TTW; j++) {
        const int tok = tok_base + 16 * j + col;
        if (tok < T) store_rows4(Y + (size_t)tok * rows, row_base + kTile * wave + 4 * g, rows,
                                 acc[j], accumulate, vec);
    }
}

// 128 rows x 64 tokens per workgroup (8 waves, one super-block per stage,
// two 64 KiB stages)
constexpr int kF16Q6RT = 8, kF16Q6TTW = 4, kF16Q6S = 2;

void launch6h(float* Y, const uint8_t* W, const uint8_t* XQ8, uint8_t* scratch, int rows, int nb,
              long row_bytes, int T, hipStream_t st, int accumulate) {
    constexpr int TW = kTile * kF16Q6TTW;
    const int Tp = (T + TW - 1) / TW * TW, nkb = nb * 8;
    auto* xh = scratch;
    auto* dxt = reinterpret_cast<float*>(xh + (size_t)nkb * Tp * 64);
    auto* gxt = dxt + (size_t)nkb * Tp;  // written by the shared re-layout, unused here
    const long n = (long)nkb * Tp;
    hipLaunchKernelGGL(k_gemm_prep16<kF16Q6TTW>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       st, XQ8, T, Tp, nkb, xh, dxt, gxt);
    const int nrt = (rows + kTile * kF16Q6RT - 1) / (kTile * kF16Q6RT);
    const unsigned grid = (unsigned)((nrt + 7) / 8 * 8 * (Tp / TW));
    hipLaunchKernelGGL((k_gemm_f16_q6k<kF16Q6RT, kF16Q6TTW, kF16Q6S>), dim3(grid),
                       dim3(kF16Q6RT * 64), 0, st, Y, W, xh, dxt, rows, nb, row_bytes, T, Tp, nrt,
                       accumulate);
}

// Tile choice: the largest of 64x64, 32x32, 16x16 (rows x tokens) whose grid
// still has one workgroup per CU; below that the 16x16 tile with the widest
// K split.  (Measured on 4096 x 11008 and 2048 x 11008 matrices, T = 8..256.)
enum class Tile6 { R64T64, R32T32, R16T16, R16T16K8 };

Tile6 pick6(int rows, int T) {
    auto grid = [&](int rw, int tw) {
        return (long)((rows + rw - 1) / rw) * (long)((T + tw - 1) / tw);
    };
    constexpr long kFill = 256;
    if (T <= 16) return Tile6::R16T16K8;
    if (grid(64, 64) >= kFill) return Tile6::R64T64;
    if (grid(32, 32) >= kFill) return Tile6::R32T32;
    if (grid(16, 16) >= kFill) return Tile6::R16T16;
    return Tile6::R16T16K8;
}

int tokens6(Tile6 t) { return t == Tile6::R64T64 ? 64 : (t == Tile6::R32T32 ? 32 : 16); }

struct MfmaCfg {
    int rt, tt;
};

// Tile choice (measured on 11008 x 4096, T = 1..64, and the 512-token
// prefill): up to 64 tokens one 16-row tile per workgroup (more workgroups in
// flight; up to 16 tokens 4 waves split the tile's sub-blocks over a 3-deep
// ring), beyond that 32 x 64 tiles.
MfmaCfg pick_mfma(int T, int nb) {
    (void)nb;
    if (T <= 16) return {1, 1};
    if (T <= 32) return {1, 2};
    return {T <= 64 ? 1 : 2, 4};
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

// bytes from W to the end of the last row's last block
static uint64_t q6k_span(int rows, int nb, long row_bytes) {
    return (uint64_t)(rows - 1) * (uint64_t)row_bytes + (uint64_t)nb * Q6K_BYTES;
}

bool gemm_mfma_q6k_ok(const void* W, int rows, int nb, long row_bytes) {
    if (rows <= 0 || nb <= 0) return false;
    const uint64_t bytes = q6k_span(rows, nb, row_bytes);
    return bytes + 16 < (1ull << 31) && ((reinterpret_cast<uintptr_t>(W) + bytes) & 15) == 0;
}

size_t gemm_mfma_q6k_scratch_bytes(int T, int nb) {
    if (T <= 0 || nb <= 0) return 0;
    const size_t tp = (size_t)((T + 63) / 64 * 64);  // the widest token tile's padding
    return (size_t)nb * 8 * tp * (64 + 4 + 4);        // fp16 re-layout (int8: 32 + 4 + 4)
}

hipError_t launch_gemm_mfma_q6k_q8(float* Y, const void* W, const void* XQ8, int rows, int T,
                                   int nb, long row_bytes, void* scratch, hipStream_t st,
                                   int accumulate) {
    if (rows <= 0 || T <= 0 || nb <= 0 || scratch == nullptr) return hipErrorInvalidValue;
    if (!gemm_mfma_q6k_ok(W, rows, nb, row_bytes)) return hipErrorInvalidValue;
    // wide token tiles on the fp16 matrix cores where 128 x 64 tiles still give
    // one workgroup per CU
    if (gemm_f16_q6k_applies(W, rows, nb, row_bytes, T)) {
        launch6h(Y, static_cast<const uint8_t*>(W), static_cast<const uint8_t*>(XQ8),
                 static_cast<uint8_t*>(scratch), rows, nb, row_bytes, T, st, accumulate);
        return hipGetLastError();
    }
    const Tile6 tile = pick6(rows, T);
    const int q = tokens6(tile);
    const int Tp = (T + q - 1) / q * q;
    const int nkb = nb * 8;
    if ((uint64_t)nkb * Tp * 32 >= (1ull << 32)) return hipErrorInvalidValue;
    auto* xs = static_cast<uint8_t*>(scratch);
    auto* dxs = reinterpret_cast<float*>(xs + (size_t)nkb * Tp * 32);
    auto* gxs = dxs + (size_t)nkb * Tp;  // written by the shared prep, unused here
    const long n = (long)nkb * Tp;
    hipLaunchKernelGGL(k_gemm_prep, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       static_cast<const uint8_t*>(XQ8), T, Tp, nkb, xs, dxs, gxs);
    const auto* w = static_cast<const uint8_t*>(W);
    switch (tile) {
    case Tile6::R64T64:
        launch6_cfg<4, 4, 2, 1, 2>(Y, w, xs, dxs, rows, nb, row_bytes, T, Tp, st, accumulate);
        break;
    case Tile6::R32T32:
        launch6_cfg<2, 2, 4, 1, 2>(Y, w, xs, dxs, rows, nb, row_bytes, T, Tp, st, accumulate);
        break;
    case Tile6::R16T16:
        launch6_cfg<1, 1, 4, 1, 2>(Y, w, xs, dxs, rows, nb, row_bytes, T, Tp, st, accumulate);
        break;
    default:
        launch6_cfg<1, 1, 8, 1, 2>(Y, w, xs, dxs, rows, nb, row_bytes, T, Tp, st, accumulate);
        break;
    }
    return hipGetLastError();
}

// 65+ tokens: the fp16 kernel, 128-row x 32-token workgroups (8 waves, two
// 36 KiB stages: two workgroups per CU), measured on the 512-token prefill
// against 64-token workgroups and 3-deep rings
constexpr int kF16MinTokens = 65;

// The fp16 GEMMs on an activation re-layout written elsewhere (the prefill's
// RMSNorm rows): xh, dxt (and gxt) as k_gemm_prep16 lays them out for Tp
// tokens (Tp a multiple of the kernel's token group: 32 for Q4_K, 64 for
// Q6_K).  Q4_K with swiglu: ffn_gate|ffn_up interleaved by 8-row blocks, the
// SwiGLU epilogue of k_gemm_f16_q4k (h as Q8_0 blocks, and fp32 rows when hf is set).
hipError_t launch_gemm_f16_q4k_xh(float* Y, uint8_t* hq8, float* hf, const void* W,
                                  const uint8_t* xh, const float* dxt, const float* gxt, int rows,
                                  int nb, long row_bytes, int T, int Tp, hipStream_t st,
                                  int accumulate, bool swiglu, uint8_t* hxh, float* hdx2,
                                  float* hgx2, float* hdx4) {
    constexpr int RT = 8, TTW = 2, S = 2, TW = kTile * TTW;
    if (rows <= 0 || nb <= 0 || T <= 0 || Tp < T || Tp % TW || (swiglu && rows % 128) ||
        (hxh && (Tp % 64 || !hdx2 || !hgx2 || !hdx4)))
        return hipErrorInvalidValue;
    const int nrt = (rows + kTile * RT - 1) / (kTile * RT);
    const unsigned grid = (unsigned)((nrt + 7) / 8 * 8 * (Tp / TW));
    const auto* w = static_cast<const uint8_t*>(W);
    if (swiglu)
        hipLaunchKernelGGL((k_gemm_f16_q4k<RT, TTW, S, true>), dim3(grid), dim3(RT * 64), 0, st,
                           nullptr, w, xh, dxt, gxt, rows, nb, row_bytes, T, Tp, nrt, 0, hq8, hf,
                           hxh, hdx2, hgx2, hdx4);
    else
        hipLaunchKernelGGL((k_gemm_f16_q4k<RT, TTW, S, false>), dim3(grid), dim3(RT * 64), 0, st,
                           Y, w, xh, dxt, gxt, rows, nb, row_bytes, T, Tp, nrt, accumulate);
    return hipGetLastError();
}

bool gemm_f16_q6k_applies(const void* W, int rows, int nb, long row_bytes, int T) {
    return T >= 64 && (long)((rows + 127) / 128) * ((T + 63) / 64) >= 256 &&
           gemm_mfma_q6k_ok(W, rows, nb, row_bytes);
}

hipError_t launch_gemm_f16_q6k_xh(float* Y, const void* W, const uint8_t* xh, const float* dxt,
                                  int rows, int nb, long row_bytes, int T, int Tp, hipStream_t st,
                                  int accumulate) {
    constexpr int TW = kTile * kF16Q6TTW;
    if (rows <= 0 || nb <= 0 || T <= 0 || Tp < T || Tp % TW || !gemm_mfma_q6k_ok(W, rows, nb, row_bytes))
        return hipErrorInvalidValue;
    const int nrt = (rows + kTile * kF16Q6RT - 1) / (kTile * kF16Q6RT);
    const unsigned grid = (unsigned)((nrt + 7) / 8 * 8 * (Tp / TW));
    hipLaunchKernelGGL((k_gemm_f16_q6k<kF16Q6RT, kF16Q6TTW, kF16Q6S>), dim3(grid),
                       dim3(kF16Q6RT * 64), 0, st, Y, static_cast<const uint8_t*>(W), xh, dxt,
                       rows, nb, row_bytes, T, Tp, nrt, accumulate);
    return hipGetLastError();
}

size_t gemm_mfma_scratch_bytes(int T, int nb) {
    if (T <= 0 || nb <= 0) return 0;
    if (T >= kF16MinTokens) {
        const size_t tp = (size_t)((T + 31) / 32 * 32);  // 32-token groups
        return (size_t)nb * 8 * tp * (64 + 4 + 4);
    }
    const size_t tp = (size_t)padded_tokens(T, pick_mfma(T, nb));
    return (size_t)nb * 8 * tp * (32 + 4 + 4);
}

// Register-weights kernel (k_gemm_q4k_rx): 4 row tiles per workgroup, K
// ranges of 4 blocks (gridDim.y of them), TT token tiles per workgroup and
// the token groups over gridDim.z.  Up to 16 tokens one tile; 17-32 two tiles
// in one group; 33-64 one tile per group (2-4 groups): on the 11008x4096
// matrix at 64 tokens 27.5 us against 29.5 us for four tiles in one group
// over 2-block K ranges (twice the split-K partials), the best of the shapes
// measured (2-8 blocks, 1-4 tiles).
constexpr int kRxRT = 4;
constexpr int kRxKB = 4;

static int rx_tt(int T) { return T > 16 && T <= 32 ? 2 : 1; }
static int rx_row_groups(int rows) { return (rows + kTile * kRxRT - 1) / (kTile * kRxRT); }
static int rx_splits(int, int nb) { return (nb + kRxKB - 1) / kRxKB; }

bool gemm_stream_q4k_ok(int T, int nb, int rows) {
    return T >= 1 && T <= kGemmStreamMaxT && nb >= 1 && rows >= 1 &&
           (size_t)T * rows < ((size_t)1 << 31);
}

size_t gemm_stream_scratch_bytes(int T, int nb, int rows) {
    if (!gemm_stream_q4k_ok(T, nb, rows) || rx_splits(T, nb) == 1) return 0;
    return (size_t)rx_splits(T, nb) * T * rows * sizeof(float);
}

hipError_t launch_gemm_stream_q4k_q8(float* Y, const void* W, const void* XQ8, int rows, int T,
                                     int nb, long row_bytes, void* scratch, hipStream_t st) {
    if (!gemm_stream_q4k_ok(T, nb, rows)) return hipErrorInvalidValue;
    // 16-byte loads of weights and activations
    if (((uintptr_t)W | (uintptr_t)XQ8 | (uintptr_t)row_bytes) & 15) return hipErrorInvalidValue;
    const int TT = rx_tt(T);
    const int S = rx_splits(T, nb);
    if (S > 1 && scratch == nullptr) return hipErrorInvalidValue;
    const int ntg = (T + kTile * TT - 1) / (kTile * TT);
    const dim3 grid((unsigned)rx_row_groups(rows), (unsigned)S, (unsigned)ntg);
    const auto* w = static_cast<const uint8_t*>(W);
    const auto* x = static_cast<const uint8_t*>(XQ8);
    auto* pt = static_cast<float*>(scratch);
    if (TT == 1)
        hipLaunchKernelGGL((k_gemm_q4k_rx<kRxRT, kRxKB, 1>), grid, dim3(kRxRT * 64), 0, st, Y, w, x, pt, rows, nb, row_bytes, T);
    else
        hipLaunchKernelGGL((k_gemm_q4k_rx<kRxRT, kRxKB, 2>), grid, dim3(kRxRT * 64), 0, st, Y, w, x, pt, rows, nb, row_bytes, T);
    if (S > 1) {
        const int n = T * rows;
        const bool vec = n % 4 == 0 && ((uintptr_t)Y & 15) == 0 && ((uintptr_t)pt & 15) == 0;
        const unsigned g4 = (unsigned)((n / 4 + 255) / 256);
        auto* Y4 = reinterpret_cast<float4*>(Y);
        const auto* P4 = reinterpret_cast<const float4*>(pt);
        if (vec && S == 2)
            hipLaunchKernelGGL(k_gemm_splitk_sum4<2>, dim3(g4), dim3(256), 0, st, Y4, P4, n / 4);
        else if (vec && S == 4)
            hipLaunchKernelGGL(k_gemm_splitk_sum4<4>, dim3(g4), dim3(256), 0, st, Y4, P4, n / 4);
        else if (vec && S == 8)
            hipLaunchKernelGGL(k_gemm_splitk_sum4<8>, dim3(g4), dim3(256), 0, st, Y4, P4, n / 4);
        else
            hipLaunchKernelGGL(k_gemm_splitk_sum, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, Y, pt, n, S);
    }
    return hipGetLastError();
}

hipError_t launch_gemm_mfma_q4k_q8(float* Y, const void* W, const void* XQ8, int rows, int T,
                                   int nb, long row_bytes, void* scratch, hipStream_t st,
                                   int accumulate) {
    if (rows <= 0 || T <= 0 || nb <= 0 || scratch == nullptr) return hipErrorInvalidValue;
    if (T >= kF16MinTokens) {
        const auto* w = static_cast<const uint8_t*>(W);
        const auto* xq = static_cast<const uint8_t*>(XQ8);
        auto* sc = static_cast<uint8_t*>(scratch);
        // 128-row tiles; 64- or 32-row tiles where those leave fewer than 256
        // workgroups (the 896-row matrices of hidden-896 models)
        const long ntg = (T + 31) / 32;
        auto wgs = [&](int rt) { return (long)((rows + kTile * rt - 1) / (kTile * rt)) * ntg; };
        if (wgs(8) >= 256)
            launch16_cfg<8, 2, 2>(Y, w, xq, sc, rows, nb, row_bytes, T, st, accumulate);
        else if (wgs(4) >= 256)
            launch16_cfg<4, 2, 2>(Y, w, xq, sc, rows, nb, row_bytes, T, st, accumulate);
        else
            launch16_cfg<2, 2, 2>(Y, w, xq, sc, rows, nb, row_bytes, T, st, accumulate);
        return hipGetLastError();
    }
    if (accumulate) return hipErrorInvalidValue;  // the int8 kernels below overwrite Y
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
    AXF_MFMA_CASE(1, 1, 4, 3)
    AXF_MFMA_CASE(1, 2, 8, 3)
    AXF_MFMA_CASE(1, 4, 8, 3)
    AXF_MFMA_CASE(2, 4, 8, 3)
    return hipErrorInvalidValue;
#undef AXF_MFMA_CASE
    return hipGetLastError();
}

}  // namespace axf
