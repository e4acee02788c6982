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
//   * partial sums are reduced over the LPR lanes with DPP row operations.
#include "common.hpp"

namespace axf {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

struct KernCfg {
    int lpr, cpl, nr;
};

// LPR lanes per row (rows of <= 16 / 32 chunks share a wave), CPL chunks per
// lane, NR rows per lane.  Every (LPR, CPL, NR) it returns is in AXF_GEMV_CFGS.
static inline KernCfg pick_cfg(int nchunks) {
    KernCfg k;
    k.lpr = nchunks <= 16 ? 16 : (nchunks <= 32 ? 32 : 64);
    k.cpl = (nchunks + k.lpr - 1) / k.lpr;
    k.nr = (k.cpl == 1 && k.lpr < 64) ? 2 : 1;
    return k;
}
#define AXF_GEMV_CFGS(X) \
    X(16, 1, 2) X(32, 1, 2) X(64, 1, 1) X(64, 2, 1) X(64, 3, 1) X(64, 4, 1) X(64, 5, 1) X(64, 6, 1) \
    X(64, 7, 1) X(64, 8, 1)
// fp32 activations above 4 chunks per lane (256 threads)
#define AXF_GEMV_CFGS_GT4(X) X(64, 5, 1) X(64, 6, 1) X(64, 7, 1) X(64, 8, 1)

// Register-prologue workgroups: two rows per lane at one chunk per lane (512
// threads), one row per lane beyond 64-lane rows of one chunk (1024 threads;
// about 32 rows per workgroup).
static inline KernCfg pick_cfg_nt(int nchunks, int nt) {
    KernCfg k = pick_cfg(nchunks);
    if (nt == 512) k.nr = k.cpl == 1 ? 2 : 1;
    if (nt == 1024) k.nr = (k.lpr == 64 && k.cpl == 1) ? 2 : 1;
    return k;
}
// Rows of 9..16 super-blocks (K 2304..4096) at 512/1024 threads run half-block
// units (PAIR): 32 lanes per row, one unit (two chunks sharing the block
// header or the Q6_K half's qh/scales) per lane, one row per 32 lanes, so a
// workgroup holds (threads / 32) rows, as many as the one-chunk layout's two
// rows per lane at 64 lanes.  Measured at 11008 x 4096 (Q4_K) and 4096 x 4096
// (Q6_K): ~9% faster than one chunk per lane; at K = 11008 it is not.
static inline bool pair_cfg(int nb) { return nb > 8 && nb <= 16; }

// K <= 8192 (fused normalisation); fp32 activations up to K = 16384 at 512
// threads and K = 12288 at 1024 (the 128-VGPR budget holds 3 Q6_K chunks per lane)
#define AXF_GEMV_CFGS_512_NORM(X) X(16, 1, 2) X(32, 1, 2) X(64, 1, 2) X(64, 2, 1) \
    X(16, 1, 1) X(32, 1, 1) X(64, 1, 1)
#define AXF_GEMV_CFGS_512(X) AXF_GEMV_CFGS_512_NORM(X) X(64, 3, 1) X(64, 4, 1)
#define AXF_GEMV_CFGS_1024_NORM(X) X(16, 1, 1) X(32, 1, 1) X(64, 1, 2) X(64, 2, 1) X(64, 1, 1)
#define AXF_GEMV_CFGS_1024(X) AXF_GEMV_CFGS_1024_NORM(X) X(64, 3, 1)
// 256 threads: one row per lane group (kShapeNR1) for Q8_0 activations; the
// fused normalisation (K <= 8192)
#define AXF_GEMV_CFGS_256_NR1(X) X(16, 1, 1) X(32, 1, 1)
#define AXF_GEMV_CFGS_256_NORM(X) X(16, 1, 2) X(32, 1, 2) X(64, 1, 1) X(64, 2, 1) \
    AXF_GEMV_CFGS_256_NR1(X)

// ---------------------------------------------------------------------------
// Activation staging
// ---------------------------------------------------------------------------

// ---------------------------------------------------------------------------
// High nibbles of four Q4_K bytes for v_dot4_i32_i8 without a shift: byte
// (q & 0xf0) ^ 0x80 read as int8 is 16*(h - 8) (one v_bitop3_b32), so a dot4
// chain over a 32-value sub-block gives 16*sum(h*x) - 128*sum(x).
// hi_dot_fix adds 128*sum(x) (the block's integer sum, which the min term
// needs anyway) and divides by 16, exactly: the result is sum(h*x).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int hi_nibbles_x16(uint32_t q) {
    return (int)((q & 0xf0f0f0f0u) ^ 0x80808080u);
}
__device__ __forceinline__ int hi_dot_fix(int dot16, int xsum) {
    return (dot16 + xsum * 128) >> 4;
}

// ---------------------------------------------------------------------------
// Q6_K byte fetch from 2-byte aligned blocks, two ways:
//   A = false: aligned dwords + v_alignbyte (more load instructions and VALU);
//   A = true:  16-byte vectors at the unaligned address (global loads take
//              them; fewer instructions, but on the 255 MB config-2 head the
//              2-byte-misaligned vectors stream ~14% slower).
// The 64-lane-row GEMVs (K >= 4096, VALU-heavy in the fused decode kernels)
// take A = true; the 16/32-lane rows (K <= 2048, bandwidth-bound) A = false.
// ---------------------------------------------------------------------------
template <int N, bool A>
__device__ __forceinline__ void load_u2(const uint8_t* p, uint32_t (&out)[N]) {
    if constexpr (A) {
        static_assert(N % 4 == 0, "whole 16-byte vectors");
#pragma unroll
        for (int k = 0; k < N / 4; k++) {
            const uint4 v = ld16_a2(p + 16 * k);
            out[4 * k] = v.x;
            out[4 * k + 1] = v.y;
            out[4 * k + 2] = v.z;
            out[4 * k + 3] = v.w;
        }
    } else {
        // reads [p & ~3, (p & ~3) + 4*(N+1)), inside the 210-byte block for the
        // ql/qh fields (N = 8)
        const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3);
        const uint8_t* base = p - sh;  // (pointer arithmetic keeps the global address space)
        uint32_t w[N + 1];
#pragma unroll
        for (int k = 0; k <= N; k++) w[k] = ld4(base + 4 * k);
#pragma unroll
        for (int k = 0; k < N; k++) out[k] = alignbyte(w[k + 1], w[k], sh);
    }
}

// Scales (16 bytes at blk+192) and d (2 bytes at blk+208), never past blk+210.
template <bool A>
__device__ __forceinline__ void load_q6_tail(const uint8_t* blk, uint32_t (&sc)[4], uint32_t& dbits) {
    if constexpr (A) {
        const uint4 v = ld16_a2(blk + 192);
        sc[0] = v.x;
        sc[1] = v.y;
        sc[2] = v.z;
        sc[3] = v.w;
        dbits = ld2(blk + 208);
    } else {
        const uint8_t* p = blk + 192;
        const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3);
        const uint8_t* base = p - sh;
        uint32_t w[5];
#pragma unroll
        for (int k = 0; k < 4; k++) w[k] = ld4(base + 4 * k);
        // sh = 2: bytes p+14..p+17 (inside the block).  sh = 0: the dword is
        // not used (alignbyte by 0 takes w[3]); it is read from p+12 so the
        // load stays inside the block, with no branch between the loads.
        w[4] = ld4(base + (sh ? 16 : 12));
        dbits = ld2(p + 16);
#pragma unroll
        for (int k = 0; k < 4; k++) sc[k] = alignbyte(w[k + 1], w[k], sh);
    }
}

// ---------------------------------------------------------------------------
// Q4_K x F32
// ---------------------------------------------------------------------------
// NT threads per workgroup: every workgroup stages the whole activation (4 KB
// per 1024 weights of a row), so larger workgroups stage it fewer times.
template <int LPR, int CPL, int NR, int NT = kThreads>
__global__ __launch_bounds__(NT) void k_gemv_q4k_f32(float* __restrict__ y,
                                                     const uint8_t* __restrict__ W,
                                                     const float* __restrict__ x, int rows,
                                                     int nb, long row_bytes, int accumulate) {
    extern __shared__ uint4 smem[];
    float* xs = reinterpret_cast<float*>(smem);
    constexpr int RPP = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rl = lane % LPR, rg = lane / LPR;
    const int nchunks = 4 * nb;
    const long row0 = ((long)blockIdx.x * (NT / 64) + wave) * (RPP * NR) + rg;

    // The first PRE float4s of x this thread stages, loaded before the
    // weights: a load issued after them could only be consumed once they had
    // all arrived (loads complete in order), and the barrier below would
    // then wait for the whole weight stream.
    constexpr int PRE = (16 * LPR * CPL + NT - 1) / NT < 4 ? (16 * LPR * CPL + NT - 1) / NT : 4;
    const int n4 = nb * (QK_K / 4);
    // (in a block of its own, so that the loads are not moved down to the
    // stores that use them)
    float4 xpre[PRE];
#pragma unroll
    for (int k = 0; k < PRE; k++) xpre[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    if ((int)threadIdx.x < n4) {
#pragma unroll
        for (int k = 0; k < PRE; k++)
            xpre[k] = reinterpret_cast<const float4*>(x)[min((int)threadIdx.x + NT * k, n4 - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);

    // weight loads from clamped (in-range) addresses, unconditional so that the
    // compiler's wait counts stay exact; chunks past the row are computed on
    // those bytes and skipped below, rows past the end are never stored
    uint4 hdr[NR][CPL], qa[NR][CPL], qb[NR][CPL];
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const long row = min(row0 + (long)n * RPP, (long)rows - 1);
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const int c = min(rl + i * LPR, nchunks - 1);
            const uint8_t* blk = W + row * row_bytes + (long)(c >> 2) * Q4K_BYTES;
            const int part = c & 3;
            hdr[n][i] = ld16(blk);
            qa[n][i] = ld16(blk + 16 + 32 * part);
            qb[n][i] = ld16(blk + 32 + 32 * part);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 64-float chunk c at float offset 68*c (an index past K rewrites the
    // last float4 with the value loaded for it, clamped above)
    if ((int)threadIdx.x < n4) {
#pragma unroll
        for (int k = 0; k < PRE; k++) {
            const int i4 = min((int)threadIdx.x + NT * k, n4 - 1);
            *reinterpret_cast<float4*>(xs + 4 * i4 + 4 * (i4 >> 4)) = xpre[k];
        }
    }
    for (int i4 = (int)threadIdx.x + NT * PRE; i4 < n4; i4 += NT) {
        const float4 v = reinterpret_cast<const float4*>(x)[i4];
        *reinterpret_cast<float4*>(xs + 4 * i4 + 4 * (i4 >> 4)) = v;
    }
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);

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
        const float v = group_sum_last<LPR>(acc[n]);
        const long row = row0 + (long)n * RPP;
        if (rl == LPR - 1 && row < rows) y[row] = accumulate ? y[row] + v : v;
    }
}

// ---------------------------------------------------------------------------
// Q6_K chunk loads: ql bytes of the chunk's two streams, the qh bytes of its
// half, the 16 scales and d, all from 2-byte-aligned block addresses.
// ---------------------------------------------------------------------------
struct Q6Chunk {
    uint32_t ql[8], qh[8], sc[4], dbits;
};

template <bool A>
__device__ __forceinline__ void load_q6_chunk(const uint8_t* blk, int c, Q6Chunk& k) {
    const int h = (c >> 1) & 1, t = c & 1;
    load_u2<8, A>(blk + 64 * h + 32 * t, k.ql);
    load_u2<8, A>(blk + 128 + 32 * h, k.qh);
    load_q6_tail<A>(blk, k.sc, k.dbits);
}

// ---------------------------------------------------------------------------
// Q8_0-activation GEMV family: Q4_K or Q6_K weights, the activation staged in
// LDS as per-chunk records, with optional fused producer / consumer work:
//   QAct::Q8    activation given as Q8_0 blocks (256-thread workgroups)
//   QAct::Norm  activation = Q8_0(w * (x * rms_scale(x))) computed by every
//               workgroup (rms_scale + q8_quant4: the same bits as
//               k_rmsnorm followed by Q8_0), so no normalisation kernel runs
//   QAct::F32   activation = Q8_0(x)
//   EPI_Y       y[row] = v, or y[row] += v (accumulate: residual adds)
//   EPI_SWIGLU  the rows of a workgroup are R/2 gate rows then R/2 up rows;
//               y[i] = swiglu(gate_i, up_i) (no SwiGLU kernel runs)
//   EPI_ARGMAX  y[row] = v, and the workgroup's largest v with its first row
//               index to pv[wg], pi[wg] (no argmax-partial kernel runs)
// Norm and F32 (K <= 16384) run 512- or 1024-thread workgroups whose threads load
// their float4s of x (and w) before issuing the weight loads, and build the
// records from registers while the weights stream in.
// Activation record of chunk c (20 dwords): int8 values of Q8_0 blocks A and
// B (8 dwords each), scales d_A and d_B, and integer sums of A and B: for
// Q4_K the sum of the 32 values (the dmin*m term), for Q6_K the sums of
// values 0-15 and 16-31 as two int16 (the -32 offset of the 6-bit weights
// under one scale per 16 weights).  Q4_K chunk c: A = 2c, B = 2c+1; Q6_K
// chunk c: A = 2c-(c&1), B = A+2.
// Weight loads use clamped (in-range) addresses; rows and chunks past the end
// are computed on those bytes and never stored.
// ---------------------------------------------------------------------------
enum { EPI_Y = 0, EPI_SWIGLU = 1, EPI_ARGMAX = 2 };
constexpr int kQ4K = AXF_TYPE_Q4_K, kQ6K = AXF_TYPE_Q6_K;
constexpr int kWide = 512, kWider = 1024;  // workgroups of the register prologue

template <int QT>
__device__ __forceinline__ uint32_t* rec_of_block(uint32_t* rec, int b, int& slot) {
    slot = QT == kQ4K ? (b & 1) : ((b >> 1) & 1);
    return rec + 20 * (QT == kQ4K ? (b >> 1) : 2 * (b >> 2) + (b & 1));
}

template <int QT>
__device__ __forceinline__ void rec_put(uint32_t* rec, int b, const uint32_t (&q)[8], float d) {
    int slot;
    uint32_t* r = rec_of_block<QT>(rec, b, slot);
    uint4* r4 = reinterpret_cast<uint4*>(r + 8 * slot);
    r4[0] = make_uint4(q[0], q[1], q[2], q[3]);
    r4[1] = make_uint4(q[4], q[5], q[6], q[7]);
    r[16 + slot] = __float_as_uint(d);
    int lo = 0, hi = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) lo = dot4((int)q[k], 0x01010101, lo);
#pragma unroll
    for (int k = 4; k < 8; k++) hi = dot4((int)q[k], 0x01010101, hi);
    r[18 + slot] = QT == kQ4K ? (uint32_t)(lo + hi) : (((uint32_t)lo & 0xffffu) | ((uint32_t)hi << 16));
}

// Token-tile staging for the dot4 GEMMs: unit u = (token t = u / nblk, Q8_0
// block b = u % nblk) of TT tokens (token t0 + min(t, nt - 1): every record
// valid).  The first PB units of a thread are loaded into registers before the
// weight loads (q8pre_load, in a block of its own so the loads are not moved
// down to their stores) and written to LDS after them (q8pre_store), so the
// workgroup barrier does not wait for the weight stream; the rest are loaded
// and written in q8pre_store.
template <int PB>
struct Q8Pre {
    uint32_t w[PB][9];  // d, then the 8 qs dwords
};
template <int PB>
__device__ __forceinline__ void q8pre_load(Q8Pre<PB>& p, const uint8_t* XQ8, size_t tok_bytes,
                                           int t0, int nt, int nblk, int total) {
#pragma unroll
    for (int k = 0; k < PB; k++)
#pragma unroll
        for (int i = 0; i < 9; i++) p.w[k][i] = 0u;
    if ((int)threadIdx.x < total) {
#pragma unroll
        for (int k = 0; k < PB; k++) {
            const int u = min((int)threadIdx.x + kThreads * k, total - 1), t = u / nblk;
            const uint8_t* b8 =
                XQ8 + (size_t)(t0 + min(t, nt - 1)) * tok_bytes + (size_t)(u - t * nblk) * Q8_0_BYTES;
#pragma unroll
            for (int i = 0; i < 9; i++) p.w[k][i] = ld4(b8 + 4 * i);
        }
    }
}
template <int QT, int PB>
__device__ __forceinline__ void q8pre_store(const Q8Pre<PB>& p, uint32_t* rec, const uint8_t* XQ8,
                                            size_t tok_bytes, int t0, int nt, int nblk, int total,
                                            int nchunks) {
    if ((int)threadIdx.x < total) {
#pragma unroll
        for (int k = 0; k < PB; k++) {
            const int u = min((int)threadIdx.x + kThreads * k, total - 1), t = u / nblk;
            const uint32_t q[8] = {p.w[k][1], p.w[k][2], p.w[k][3], p.w[k][4],
                                   p.w[k][5], p.w[k][6], p.w[k][7], p.w[k][8]};
            rec_put<QT>(rec + (size_t)t * 20 * nchunks, u - t * nblk, q, __uint_as_float(p.w[k][0]));
        }
    }
    for (int u = (int)threadIdx.x + kThreads * PB; u < total; u += kThreads) {
        const int t = u / nblk;
        const uint8_t* b8 =
            XQ8 + (size_t)(t0 + min(t, nt - 1)) * tok_bytes + (size_t)(u - t * nblk) * Q8_0_BYTES;
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = ld4(b8 + 4 + 4 * i);
        rec_put<QT>(rec + (size_t)t * 20 * nchunks, u - t * nblk, q, __uint_as_float(ld4(b8)));
    }
}

// Staging: one Q8_0 block per thread and step.  With Q8_0 input the block of
// the first step (b = threadIdx.x) was loaded into pre[] (d, 8 qs dwords)
// before the weight loads, so it is staged while the weights stream in (a
// load issued after them could only be consumed once they had all arrived:
// loads complete in order); the blocks of later steps (K > 32 * NT) are
// loaded here.
template <int QT, int NT, int ACT>
__device__ __forceinline__ void stage_act(uint32_t* rec, const QGemvArgs& a,
                                          const uint32_t (&pre)[9]) {
    const int nblk = a.nb * QK_K / 32;
    int b0 = threadIdx.x;
    if (ACT == (int)QAct::Q8) {
        if (b0 < nblk) {
            const uint32_t q[8] = {pre[1], pre[2], pre[3], pre[4], pre[5], pre[6], pre[7], pre[8]};
            rec_put<QT>(rec, b0, q, __uint_as_float(pre[0]));
        }
        b0 += NT;
    }
    for (int b = b0; b < nblk; b += NT) {
        uint32_t q[8];
        float d;
        if (ACT == (int)QAct::Q8) {
            const uint8_t* p = a.xq8 + (size_t)b * Q8_0_BYTES;
#pragma unroll
            for (int k = 0; k < 8; k++) q[k] = ld4(p + 4 + 4 * k);
            d = __uint_as_float(ld4(p));
        } else {
            const float4* xp = reinterpret_cast<const float4*>(a.x + 32 * (size_t)b);
            float v[32];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float4 t = xp[k];
                v[4 * k] = t.x;
                v[4 * k + 1] = t.y;
                v[4 * k + 2] = t.z;
                v[4 * k + 3] = t.w;
            }
            q8_quant32(v, q, d);
        }
        rec_put<QT>(rec, b, q, d);
    }
}

// Staging from registers: thread t holds float4 t + NT*k of x (and w); 8
// consecutive threads hold one Q8_0 block.
template <int QT, int NT, int KPT, int ACT>
__device__ __forceinline__ void stage_regs(uint32_t* rec, float4 (&xv)[KPT],
                                           const float4 (&wv)[KPT], int n4, float eps,
                                           float* red) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < KPT; k++)
        if (tid + NT * k >= n4) xv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    float rs = 1.f;
    if (ACT == (int)QAct::Norm) rs = rms_scale<NT, KPT>(xv, 4 * n4, eps, red);
#pragma unroll
    for (int k = 0; k < KPT; k++) {
        const int i4 = tid + NT * k;
        float4 v = xv[k];
        if (ACT == (int)QAct::Norm) {
            const float4 g = wv[k];
            v = make_float4(g.x * (v.x * rs), g.y * (v.y * rs), g.z * (v.z * rs), g.w * (v.w * rs));
        }
        float d;
        const uint32_t q = q8_quant4(v, d);
        // integer sums over the block (Q4_K) or its two halves (Q6_K)
        const int s = sum_quad(dot4((int)q, 0x01010101, 0));
        const int s_hi = half_mirror(s);  // lane sub 0 receives the sum of lanes 4-7
        const int sub = i4 & 7;
        if (i4 < n4) {
            int slot;
            uint32_t* r = rec_of_block<QT>(rec, i4 >> 3, slot);
            r[8 * slot + sub] = q;
            if (sub == 0) {
                r[16 + slot] = __float_as_uint(d);
                r[18 + slot] = QT == kQ4K ? (uint32_t)(s + s_hi)
                                          : (((uint32_t)s & 0xffffu) | ((uint32_t)s_hi << 16));
            }
        }
    }
}

// Integer sums of a directly loaded record (dx[0..1] block A, dx[2..3] block
// B) into dx[4].z / .w, encoded as in rec_put.
template <int QT>
__device__ __forceinline__ void direct_sums(uint4 (&dx)[5]) {
    const uint32_t a[8] = {dx[0].x, dx[0].y, dx[0].z, dx[0].w, dx[1].x, dx[1].y, dx[1].z, dx[1].w};
    const uint32_t b[8] = {dx[2].x, dx[2].y, dx[2].z, dx[2].w, dx[3].x, dx[3].y, dx[3].z, dx[3].w};
    int alo = 0, ahi = 0, blo = 0, bhi = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        alo = dot4((int)a[k], 0x01010101, alo);
        ahi = dot4((int)a[k + 4], 0x01010101, ahi);
        blo = dot4((int)b[k], 0x01010101, blo);
        bhi = dot4((int)b[k + 4], 0x01010101, bhi);
    }
    if (QT == kQ4K) {
        dx[4].z = (uint32_t)(alo + ahi);
        dx[4].w = (uint32_t)(blo + bhi);
    } else {
        dx[4].z = ((uint32_t)alo & 0xffffu) | ((uint32_t)ahi << 16);
        dx[4].w = ((uint32_t)blo & 0xffffu) | ((uint32_t)bhi << 16);
    }
}

// One Q4_K chunk (64 weights: sub-blocks 2*part, 2*part+1, qs bytes qa|qb)
// of one row against its activation record (xa, xb, meta = {d_A, d_B, sum_A,
// sum_B}); returns acc plus the chunk's contribution.
__device__ __forceinline__ float q4k_chunk_dot(float acc, const uint4& h, const uint4& qa,
                                               const uint4& qb, int part,
                                               const uint32_t (&xa)[8], const uint32_t (&xb)[8],
                                               const uint4& meta) {
    const float dx0 = __uint_as_float(meta.x), dx1 = __uint_as_float(meta.y);
    const float sx0 = (float)(int)meta.z, sx1 = (float)(int)meta.w;
    const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
    uint32_t sc0, m0, sc1, m1;
    q4k_scales(h.y, h.z, h.w, part, sc0, m0, sc1, m1);
    const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    int dlo = 0, dhi = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        dlo = dot4((int)(q[k] & 0x0f0f0f0fu), (int)xa[k], dlo);
        dhi = dot4(hi_nibbles_x16(q[k]), (int)xb[k], dhi);
    }
    dhi = hi_dot_fix(dhi, (int)meta.w);
    const float s0 = ((float)sc0 * d) * dx0, mm0 = ((float)m0 * dmin) * dx0;
    const float s1 = ((float)sc1 * d) * dx1, mm1 = ((float)m1 * dmin) * dx1;
    float v = acc;
    v = fmaf(s0, (float)dlo, v);
    v = fmaf(-mm0, sx0, v);
    v = fmaf(s1, (float)dhi, v);
    v = fmaf(-mm1, sx1, v);
    return v;
}

// One Q6_K chunk t of a half block: ql = its 8 ql dwords (low nibbles: part
// t, high nibbles: part t+2), qh = the half's 8 qh dwords, sa / sb = the
// half's scale bytes 0-3 / 4-7, d the block scale.  The -32 offset comes from
// the record's per-16 activation sums.
__device__ __forceinline__ float q6k_chunk_dot(float acc, const uint32_t* ql, const uint32_t* qh,
                                               int t, uint32_t sa, uint32_t sb, float d,
                                               const uint32_t (&xa)[8], const uint32_t (&xb)[8],
                                               const uint4& meta) {
    const float dxa = __uint_as_float(meta.x), dxb = __uint_as_float(meta.y);
    const int sA0 = (int8_t)(sa >> (16 * t)), sA1 = (int8_t)(sa >> (16 * t + 8));
    const int sB0 = (int8_t)(sb >> (16 * t)), sB1 = (int8_t)(sb >> (16 * t + 8));
    int iA0 = -32 * (int)(int16_t)(meta.z & 0xffffu), iA1 = -32 * ((int)meta.z >> 16);
    int iB0 = -32 * (int)(int16_t)(meta.w & 0xffffu), iB1 = -32 * ((int)meta.w >> 16);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t l = ql[k], hs = qh[k] >> (2 * t);
        // 6-bit values: low nibble from ql, bits 4-5 from qh
        const uint32_t qA = (l & 0x0f0f0f0fu) | ((hs << 4) & 0x30303030u);
        const uint32_t qB = ((l >> 4) & 0x0f0f0f0fu) | (hs & 0x30303030u);
        if (k < 4) {
            iA0 = dot4((int)qA, (int)xa[k], iA0);
            iB0 = dot4((int)qB, (int)xb[k], iB0);
        } else {
            iA1 = dot4((int)qA, (int)xa[k], iA1);
            iB1 = dot4((int)qB, (int)xb[k], iB1);
        }
    }
    float v = acc;
    v = fmaf((d * (float)sA0) * dxa, (float)iA0, v);
    v = fmaf((d * (float)sA1) * dxa, (float)iA1, v);
    v = fmaf((d * (float)sB0) * dxb, (float)iB0, v);
    v = fmaf((d * (float)sB1) * dxb, (float)iB1, v);
    return v;
}

__device__ __forceinline__ void rec_load(const uint32_t* rec, int c, uint32_t (&xa)[8],
                                         uint32_t (&xb)[8], uint4& meta) {
    const uint4* r4 = reinterpret_cast<const uint4*>(rec + 20 * c);
    const uint4 a0 = r4[0], a1 = r4[1], b0 = r4[2], b1 = r4[3];
    meta = r4[4];
    xa[0] = a0.x; xa[1] = a0.y; xa[2] = a0.z; xa[3] = a0.w;
    xa[4] = a1.x; xa[5] = a1.y; xa[6] = a1.z; xa[7] = a1.w;
    xb[0] = b0.x; xb[1] = b0.y; xb[2] = b0.z; xb[3] = b0.w;
    xb[4] = b1.x; xb[5] = b1.y; xb[6] = b1.z; xb[7] = b1.w;
}

// Work units: PAIR = false: a unit is one chunk, lane (rl, i) owns chunk
// rl + i*LPR.  PAIR = true: a unit is half a super-block (chunks 2u, 2u+1,
// 128 weights), lane (rl, i) owns unit u = rl + i*LPR; the two chunks share
// the block header (Q4_K d, dmin, scales) or the half's qh bytes, scales and d
// (Q6_K), which are loaded and decoded once.  CPL counts units per lane.
typedef __attribute__((address_space(1))) const void gmem_t;
typedef __attribute__((address_space(3))) void lmem_t;

template <int QT, int NT, int LPR, int CPL, int NR, int ACT, int EPI, bool PAIR, bool WL = false>
__device__ __forceinline__ void qgemv_body(const QGemvArgs& a, const uint8_t* __restrict__ W,
                                           long rb, int rows, float* __restrict__ y, int wg,
                                           uint32_t* rec, float* red, uint8_t* wlds = nullptr) {
    constexpr int RPP = 64 / LPR;
    constexpr int RW = (NT / 64) * RPP * NR;  // rows per workgroup
    constexpr int UC = PAIR ? 2 : 1;          // chunks per unit
    // activation built from registers: the fused normalisation, and fp32 at 512+ threads
    constexpr bool REG = ACT == (int)QAct::Norm || (NT >= kWide && ACT == (int)QAct::F32);
    // the one-chunk Q6_K rows with an fp32 activation at 512+ threads (the
    // decode down-projection): only the first unit's weights are issued before
    // the activation is staged, the rest after, so the activation's registers
    // are free before most of the weights' go live: 111 -> 94 VGPRs, two
    // 512-thread workgroups resident per CU instead of one.  7B down 14.05 ->
    // 12.95 us, decode step 1.783 -> 1.771 ms, config-3 step 41.6 -> 41.2 us
    // (staging before any weight load: 13.85 us, 1.779 ms; that with
    // 1024-thread workgroups: 1.787 ms)
    constexpr bool SFIRST = QT == kQ6K && ACT == (int)QAct::F32 && NT >= kWide && !PAIR;
    // WL (Q6_K half-block units, rows of a multiple of 16 bytes): the wave's
    // RPP*NR consecutive rows are copied into LDS by 16-byte global_load_lds
    // (64 lanes x 16 B of one contiguous span per instruction) and the lanes
    // read their units' fields from there, instead of ~28 scattered dword
    // loads per lane from global memory
    static_assert(!WL || (QT == kQ6K && PAIR), "LDS-staged weights: Q6_K half-block units");
    // float4s of x per thread: K / 4 <= 16 * LPR * CPL * UC
    constexpr int KPT = (16 * LPR * CPL * UC + NT - 1) / NT;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rl = lane % LPR, rg = lane / LPR;
    const int nunits = 4 * a.nb / UC;
    const int rloc0 = wave * (RPP * NR) + rg;
    const long row0 = (long)wg * RW + rloc0;
    float acc[NR];
#pragma unroll
    for (int n = 0; n < NR; n++) acc[n] = 0.f;

    // One chunk per lane with Q8_0 input: each lane reads its chunk's two Q8_0
    // blocks itself (L2-resident), before its weight loads; no LDS staging.
    constexpr bool DIRECT = ACT == (int)QAct::Q8 && CPL == 1 && NT == kThreads && !PAIR;
    uint4 dx[5];  // the chunk's activation record (DIRECT)
    if constexpr (DIRECT) {
        const int c = min(rl, nunits - 1);
        const int A = QT == kQ4K ? 2 * c : 2 * c - (c & 1);
        const int B = QT == kQ4K ? A + 1 : A + 2;
        const uint8_t* pa = a.xq8 + (size_t)A * Q8_0_BYTES;
        const uint8_t* pb = a.xq8 + (size_t)B * Q8_0_BYTES;
        dx[0] = make_uint4(ld4(pa + 4), ld4(pa + 8), ld4(pa + 12), ld4(pa + 16));
        dx[1] = make_uint4(ld4(pa + 20), ld4(pa + 24), ld4(pa + 28), ld4(pa + 32));
        dx[2] = make_uint4(ld4(pb + 4), ld4(pb + 8), ld4(pb + 12), ld4(pb + 16));
        dx[3] = make_uint4(ld4(pb + 20), ld4(pb + 24), ld4(pb + 28), ld4(pb + 32));
        dx[4] = make_uint4(ld4(pa), ld4(pb), 0u, 0u);
        __builtin_amdgcn_sched_barrier(0);
    }
    // Q8_0 input staged through LDS: this thread's first block, ahead of the weights
    uint32_t pre[9];
    if constexpr (ACT == (int)QAct::Q8 && !DIRECT) {
        if ((int)threadIdx.x < a.nb * (QK_K / 32)) {
            const uint8_t* p = a.xq8 + (size_t)threadIdx.x * Q8_0_BYTES;
#pragma unroll
            for (int k = 0; k < 9; k++) pre[k] = ld4(p + 4 * k);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    float4 xv[KPT], wv[KPT];
    const int n4 = a.nb * (QK_K / 4);
    // embedding row (QAct::Norm with a.emb): per float4, the Q4_K block header
    // and the dword of 4 nibbles, decoded once the weight loads are in flight
    const bool emb = ACT == (int)QAct::Norm && a.emb != nullptr;
    uint4 eh[ACT == (int)QAct::Norm ? KPT : 1];
    uint32_t eq[ACT == (int)QAct::Norm ? KPT : 1];
    if constexpr (REG) {
        if (ACT == (int)QAct::Norm && emb) {
            const int id = a.tok_dev ? *a.tok_dev : a.tok;
            const uint8_t* er = a.emb + (long)id * a.emb_rb;
#pragma unroll
            for (int k = 0; k < KPT; k++) {
                const int i4 = min((int)threadIdx.x + NT * k, n4 - 1);
                const uint8_t* blk = er + (long)(i4 >> 6) * Q4K_BYTES;
                // elements 4*i4 .. +3: chunk (i4 >> 4) & 3, nibble run (i4 >> 3) & 1
                eh[k] = ld16(blk);
                eq[k] = ld4(blk + 16 + 32 * ((i4 >> 4) & 3) + 4 * (i4 & 7));
                wv[k] = reinterpret_cast<const float4*>(a.nw)[i4];
            }
        } else {
#pragma unroll
            for (int k = 0; k < KPT; k++) {
                const int i4 = min((int)threadIdx.x + NT * k, n4 - 1);
                xv[k] = reinterpret_cast<const float4*>(a.x)[i4];
                wv[k] = ACT == (int)QAct::Norm ? reinterpret_cast<const float4*>(a.nw)[i4]
                                               : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    // the activation, once this lane's weight loads are in flight
    auto stage = [&]() {
        if constexpr (REG && ACT == (int)QAct::Norm) {
            if (emb) {
                // k_embed_q4k's arithmetic: fmaf(d*sc, q, -(dmin*m)) per element
#pragma unroll
                for (int k = 0; k < KPT; k++) {
                    const int i4 = (int)threadIdx.x + NT * k;
                    const int c = (i4 >> 4) & 3, hi = (i4 >> 3) & 1;
                    const float d = h2f(eh[k].x & 0xffffu), dmin = h2f(eh[k].x >> 16);
                    uint32_t sc0, m0, sc1, m1;
                    q4k_scales(eh[k].y, eh[k].z, eh[k].w, c, sc0, m0, sc1, m1);
                    const float ds = d * (float)(hi ? sc1 : sc0), dm = dmin * (float)(hi ? m1 : m0);
                    const uint32_t q = hi ? eq[k] >> 4 : eq[k];
                    xv[k] = make_float4(fmaf(ds, (float)(q & 0xfu), -dm),
                                        fmaf(ds, (float)((q >> 8) & 0xfu), -dm),
                                        fmaf(ds, (float)((q >> 16) & 0xfu), -dm),
                                        fmaf(ds, (float)((q >> 24) & 0xfu), -dm));
                    if (blockIdx.x == 0 && i4 < n4) reinterpret_cast<float4*>(a.x_out)[i4] = xv[k];
                }
            }
        }
        if constexpr (DIRECT)
            direct_sums<QT>(dx);
        else if constexpr (REG)
            stage_regs<QT, NT, KPT, ACT>(rec, xv, wv, n4, a.eps, red);
        else
            stage_act<QT, NT, ACT>(rec, a, pre);
        if constexpr (!DIRECT) __syncthreads();
    };

    if constexpr (QT == kQ4K) {
        // unit (n, i): header, then 16-byte qs vectors (2 per chunk)
        uint4 hdr[NR][CPL], qv[NR][CPL][2 * UC];
#pragma unroll
        for (int n = 0; n < NR; n++) {
            const long row = min(row0 + (long)n * RPP, (long)rows - 1);
#pragma unroll
            for (int i = 0; i < CPL; i++) {
                const int u = min(rl + i * LPR, nunits - 1);
                const uint8_t* blk = W + row * rb + (long)(u * UC >> 2) * Q4K_BYTES;
                // first qs byte of the unit: 32 * part (chunk) or 64 * half (pair)
                const int q0 = 16 + (PAIR ? 64 * (u & 1) : 32 * (u & 3));
                hdr[n][i] = ld16(blk);
#pragma unroll
                for (int k = 0; k < 2 * UC; k++) qv[n][i][k] = ld16(blk + q0 + 16 * k);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        stage();
        // nothing that waits for the weights above the workgroup barrier
        __builtin_amdgcn_sched_barrier(0);
        // every unit is computed on clamped (valid) data and its contribution
        // selected, so no load is sunk into a branch
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const bool live = rl + i * LPR < nunits;
            const int u = min(rl + i * LPR, nunits - 1);
#pragma unroll
            for (int j = 0; j < UC; j++) {
                const int c = u * UC + j;
                uint32_t xa[8], xb[8];
                uint4 meta;
                if constexpr (DIRECT) {
                    const uint4 r[4] = {dx[0], dx[1], dx[2], dx[3]};
                    xa[0] = r[0].x; xa[1] = r[0].y; xa[2] = r[0].z; xa[3] = r[0].w;
                    xa[4] = r[1].x; xa[5] = r[1].y; xa[6] = r[1].z; xa[7] = r[1].w;
                    xb[0] = r[2].x; xb[1] = r[2].y; xb[2] = r[2].z; xb[3] = r[2].w;
                    xb[4] = r[3].x; xb[5] = r[3].y; xb[6] = r[3].z; xb[7] = r[3].w;
                    meta = dx[4];
                } else {
                    rec_load(rec, c, xa, xb, meta);
                }
                const int part = c & 3;
#pragma unroll
                for (int n = 0; n < NR; n++) {
                    const float v = q4k_chunk_dot(acc[n], hdr[n][i], qv[n][i][2 * j],
                                                  qv[n][i][2 * j + 1], part, xa, xb, meta);
                    acc[n] = live ? v : acc[n];
                }
            }
        }
    } else {
        // unit (n, i): ql (8 dwords per chunk), the half's qh (8 dwords), scales, d
        uint32_t ql[NR][CPL][8 * UC], qh[NR][CPL][8], sc[NR][CPL][4], db[NR][CPL];
        const int wv_ = __builtin_amdgcn_readfirstlane(wave);
        uint8_t* wl = wlds + (size_t)wv_ * (RPP * NR) * rb;  // this wave's rows in LDS
        if constexpr (WL) {
            // rows wg*RW + wave*RPP*NR .. +RPP*NR-1; past the matrix end the
            // addresses are clamped to its last 16 bytes (rows never stored)
            const long first = (long)wg * RW + (long)wv_ * (RPP * NR);
            const int span = (RPP * NR) * (int)rb;
            const uint8_t* g0 = W + first * rb;
            const uint8_t* gend = W + (long)rows * rb - 16;
            for (int o = 0; o < span; o += 1024) {
                const int lo = o + 16 * lane;
                const uint8_t* g = g0 + lo;
                if (lo < span)
                    __builtin_amdgcn_global_load_lds((gmem_t*)(g < gend ? g : gend),
                                                     (lmem_t*)(wl + o), 16, 0, 0);
            }
        }
        auto load6 = [&](int n, int i) {
            const long row = min(row0 + (long)n * RPP, (long)rows - 1);
            const int u = min(rl + i * LPR, nunits - 1);
            const int c0 = u * UC;  // first chunk of the unit
            const int h = (c0 >> 1) & 1, t = c0 & 1;
            const uint8_t* blk = WL ? wl + (long)(rloc0 - wv_ * (RPP * NR) + n * RPP) * rb +
                                          (long)(c0 >> 2) * Q6K_BYTES
                                    : W + row * rb + (long)(c0 >> 2) * Q6K_BYTES;
            if constexpr (PAIR) {
                // 64 ql bytes, 32 qh bytes, 8 scale bytes of half h, and d, as
                // aligned dwords + v_alignbyte: against 16-byte vectors at the
                // 2-byte aligned addresses, 9.4 -> 9.2 us for the 7B q|k|v
                // launch and 26.7 -> 24.9 us for the 32000 x 4096 head (the
                // K = 11008 one-chunk rows measured the other way: 14.0 -> 14.7 us)
                load_u2<16, false>(blk + 64 * h, ql[n][i]);
                load_u2<8, false>(blk + 128 + 32 * h, qh[n][i]);
                {
                    // 8 bytes at blk + 192 + 8h; the third dword is read only when
                    // the field is 2 bytes past a dword (it then ends at blk + 210)
                    const uint8_t* p = blk + 192 + 8 * h;
                    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3);
                    const uint8_t* base = p - sh;
                    const uint32_t w0 = ld4(base), w1 = ld4(base + 4);
                    const uint32_t w2 = ld4(base + (sh ? 8 : 4));
                    sc[n][i][0] = alignbyte(w1, w0, sh);
                    sc[n][i][1] = alignbyte(w2, w1, sh);
                }
                sc[n][i][2] = sc[n][i][3] = 0u;
                db[n][i] = ld2(blk + 208);
            } else {
                load_u2<8, LPR == 64>(blk + 64 * h + 32 * t, ql[n][i]);
                load_u2<8, LPR == 64>(blk + 128 + 32 * h, qh[n][i]);
                load_q6_tail<LPR == 64>(blk, sc[n][i], db[n][i]);
            }
        };
        if constexpr (WL) {
            // the copies are in flight during the activation staging; each wave
            // reads only its own rows, so its own wait suffices
            stage();
            __builtin_amdgcn_s_waitcnt(0xf70);  // vmcnt(0) (gfx9 encoding, lgkm/exp at maxima)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int n = 0; n < NR; n++)
#pragma unroll
                for (int i = 0; i < CPL; i++) load6(n, i);
        } else if constexpr (SFIRST) {
            // the first unit's weights in flight during the staging
#pragma unroll
            for (int n = 0; n < NR; n++) load6(n, 0);
            __builtin_amdgcn_sched_barrier(0);
            stage();
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int n = 0; n < NR; n++)
#pragma unroll
                for (int i = 1; i < CPL; i++) load6(n, i);
        } else {
#pragma unroll
            for (int n = 0; n < NR; n++)
#pragma unroll
                for (int i = 0; i < CPL; i++) load6(n, i);
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (!SFIRST && !WL) stage();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const bool live = rl + i * LPR < nunits;
            const int u = min(rl + i * LPR, nunits - 1);
#pragma unroll
            for (int j = 0; j < UC; j++) {
                const int c = u * UC + j;
                uint32_t xa[8], xb[8];
                uint4 meta;
                if constexpr (DIRECT) {
                    const uint4 r[4] = {dx[0], dx[1], dx[2], dx[3]};
                    xa[0] = r[0].x; xa[1] = r[0].y; xa[2] = r[0].z; xa[3] = r[0].w;
                    xa[4] = r[1].x; xa[5] = r[1].y; xa[6] = r[1].z; xa[7] = r[1].w;
                    xb[0] = r[2].x; xb[1] = r[2].y; xb[2] = r[2].z; xb[3] = r[2].w;
                    xb[4] = r[3].x; xb[5] = r[3].y; xb[6] = r[3].z; xb[7] = r[3].w;
                    meta = dx[4];
                } else {
                    rec_load(rec, c, xa, xb, meta);
                }
                const int h = (c >> 1) & 1, t = c & 1;
#pragma unroll
                for (int n = 0; n < NR; n++) {
                    // PAIR: the scale dwords are the half's; otherwise all 16 scales
                    // (selected by mask, not by a runtime array index)
                    const uint32_t hm = PAIR ? 0u : 0u - (uint32_t)h;
                    const uint32_t sa = sc[n][i][0] ^ ((sc[n][i][0] ^ sc[n][i][2]) & hm);
                    const uint32_t sb = sc[n][i][1] ^ ((sc[n][i][1] ^ sc[n][i][3]) & hm);
                    const float v = q6k_chunk_dot(acc[n], &ql[n][i][8 * j], qh[n][i], t, sa, sb,
                                                  h2f(db[n][i]), xa, xb, meta);
                    acc[n] = live ? v : acc[n];
                }
            }
        }
    }

    if constexpr (EPI == EPI_Y) {
#pragma unroll
        for (int n = 0; n < NR; n++) {
            const float v = group_sum_last<LPR>(acc[n]);
            const long row = row0 + (long)n * RPP;
            if (rl == LPR - 1 && row < rows) y[row] = a.accumulate ? y[row] + v : v;
        }
    } else if constexpr (EPI == EPI_ARGMAX) {
        static_assert(RW <= 64, "one wave merges the workgroup's rows");
        float* hv = red + 16;  // the RW row results of this workgroup
#pragma unroll
        for (int n = 0; n < NR; n++) {
            const float v = group_sum_last<LPR>(acc[n]);
            const long row = row0 + (long)n * RPP;
            if (rl == LPR - 1) {
                if (row < rows) y[row] = v;
                hv[rloc0 + n * RPP] = v;
            }
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            // the argmax merge: a larger value wins, an equal value with a
            // smaller index wins, NaN never wins; from (-inf, INT_MAX), so a
            // workgroup of NaN rows reports (-inf, INT_MAX)
            float bv = -INFINITY;
            int bi = 0x7fffffff;
            const int row = wg * RW + (int)threadIdx.x;
            if ((int)threadIdx.x < RW && row < rows) {
                const float v = hv[threadIdx.x];
                if (v > bv || v == bv) {
                    bv = v;
                    bi = row;
                }
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                const float v2 = __shfl_xor(bv, off, 64);
                const int i2 = __shfl_xor(bi, off, 64);
                if (v2 > bv || (v2 == bv && i2 < bi)) {
                    bv = v2;
                    bi = i2;
                }
            }
            if (threadIdx.x == 0) {
                a.pv[wg] = bv;
                a.pi[wg] = bi;
            }
        }
    } else {
        float* hv = red + 16;  // RW row results of this workgroup
#pragma unroll
        for (int n = 0; n < NR; n++) {
            const float v = group_sum_last<LPR>(acc[n]);
            if (rl == LPR - 1) hv[rloc0 + n * RPP] = v;
        }
        __syncthreads();
        if ((int)threadIdx.x < RW / 2) {
            const long i = (long)wg * (RW / 2) + threadIdx.x;
            if (2 * i < rows) y[i] = swiglu1(hv[threadIdx.x], hv[RW / 2 + threadIdx.x]);
        }
    }
}

template <int QT, int NT, int LPR, int CPL, int NR, int ACT, int EPI, bool PAIR, bool WL = false>
__global__ __launch_bounds__(NT) void k_qgemv(QGemvArgs a) {
    extern __shared__ uint4 smem[];
    uint32_t* rec = reinterpret_cast<uint32_t*>(smem);
    float* red = reinterpret_cast<float*>(rec + 80 * a.nb);
    // WL: the weight rows after rec and red (qgemv_lds, 16-byte aligned)
    uint8_t* wl = reinterpret_cast<uint8_t*>(smem) + 320 * a.nb + 4 * (16 + 256);
    qgemv_body<QT, NT, LPR, CPL, NR, ACT, EPI, PAIR, WL>(a, a.W0, a.rb0, a.rows0, a.y0,
                                                          blockIdx.x, rec, red, wl);
}

// Workgroups [0, nwg0) run the Q4_K segment, the rest the Q6_K segment.
template <int NT, int LPR, int CPL, int NR, int ACT, bool PAIR>
__global__ __launch_bounds__(NT) void k_qgemv2(QGemvArgs a) {
    extern __shared__ uint4 smem[];
    uint32_t* rec = reinterpret_cast<uint32_t*>(smem);
    float* red = reinterpret_cast<float*>(rec + 80 * a.nb);
    if ((int)blockIdx.x < a.nwg0)
        qgemv_body<kQ4K, NT, LPR, CPL, NR, ACT, EPI_Y, PAIR>(a, a.W0, a.rb0, a.rows0, a.y0,
                                                              blockIdx.x, rec, red);
    else
        qgemv_body<kQ6K, NT, LPR, CPL, NR, ACT, EPI_Y, PAIR>(a, a.W1, a.rb1, a.rows1, a.y1,
                                                              blockIdx.x - a.nwg0, rec, red);
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

    // the first PRE float4s of x this thread stages, ahead of the weights (as
    // in k_gemv_q4k_f32)
    constexpr int PRE = (16 * LPR * CPL + kThreads - 1) / kThreads < 4
                            ? (16 * LPR * CPL + kThreads - 1) / kThreads : 4;
    const int n4 = nb * (QK_K / 4);
    float4 xpre[PRE];
#pragma unroll
    for (int k = 0; k < PRE; k++) xpre[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    if ((int)threadIdx.x < n4) {
#pragma unroll
        for (int k = 0; k < PRE; k++)
            xpre[k] = reinterpret_cast<const float4*>(x)[min((int)threadIdx.x + kThreads * k, n4 - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);

    // unconditional loads from clamped addresses (as in k_gemv_q4k_f32)
    Q6Chunk wk[NR][CPL];
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const long row = min(row0 + (long)n * RPP, (long)rows - 1);
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const int c = min(rl + i * LPR, nchunks - 1);
            load_q6_chunk<LPR == 64>(W + row * row_bytes + (long)(c >> 2) * Q6K_BYTES, c, wk[n][i]);
        }
    }

    __builtin_amdgcn_sched_barrier(0);
    // 32-float part p at float offset 36*p
    if ((int)threadIdx.x < n4) {
#pragma unroll
        for (int k = 0; k < PRE; k++) {
            const int i4 = min((int)threadIdx.x + kThreads * k, n4 - 1);
            *reinterpret_cast<float4*>(xs + 4 * i4 + 4 * (i4 >> 3)) = xpre[k];
        }
    }
    for (int i4 = (int)threadIdx.x + kThreads * PRE; i4 < n4; i4 += kThreads) {
        const float4 v = reinterpret_cast<const float4*>(x)[i4];
        *reinterpret_cast<float4*>(xs + 4 * i4 + 4 * (i4 >> 3)) = v;
    }
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);

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
        const float v = group_sum_last<LPR>(acc[n]);
        const long row = row0 + (long)n * RPP;
        if (rl == LPR - 1 && row < rows) y[row] = accumulate ? y[row] + v : v;
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
    const int nblk = 8 * nb, total = TT * nblk;
    Q8Pre<2> pre;
    q8pre_load(pre, XQ8, tok_bytes, t0, nt, nblk, total);
    __builtin_amdgcn_sched_barrier(0);

    // weight loads from clamped addresses, unconditional (exact wait counts);
    // chunks past the row are skipped below, rows past the end never stored
    uint4 hdr[NR][CPL], qa[NR][CPL], qb[NR][CPL];
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const long row = min(row0 + (long)n * RPP, (long)rows - 1);
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const int c = min(rl + i * LPR, nchunks - 1);
            const uint8_t* blk = W + row * row_bytes + (long)(c >> 2) * Q4K_BYTES;
            const int part = c & 3;
            hdr[n][i] = ld16(blk);
            qa[n][i] = ld16(blk + 16 + 32 * part);
            qb[n][i] = ld16(blk + 32 + 32 * part);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    q8pre_store<kQ4K>(pre, rec, XQ8, tok_bytes, t0, nt, nblk, total, nchunks);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);

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
                            dhi = dot4(hi_nibbles_x16(q[k]), (int)xb[k], dhi);
                        }
                        dhi = hi_dot_fix(dhi, (int)meta.w);
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
            const float v = group_sum_last<LPR>(acc[n][t]);
            if (rl == LPR - 1 && row < rows && t < nt) Y[(size_t)(t0 + t) * rows + row] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Batched Q6_K x Q8_0 (small M): Y[t*rows + o] for a tile of TT tokens.  The
// reference runs one gemv_q6k_q8_avx2_range per token for Q6_K weights
// (gemm_wt_q8, src/models/llama_model.cpp:860-873); here each lane decodes its
// weight chunks once and applies them to the TT tokens' records in LDS (the
// GEMV's lane decomposition and per-chunk arithmetic).
// ---------------------------------------------------------------------------
template <int LPR, int CPL, int NR, int TT>
__global__ __launch_bounds__(kThreads) void k_gemm_q6k_q8(float* __restrict__ Y,
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
    const int nblk = 8 * nb, total = TT * nblk;
    Q8Pre<2> pre;
    q8pre_load(pre, XQ8, tok_bytes, t0, nt, nblk, total);
    __builtin_amdgcn_sched_barrier(0);

    Q6Chunk wk[NR][CPL];
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const long row = min(row0 + (long)n * RPP, (long)rows - 1);
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const int c = min(rl + i * LPR, nchunks - 1);
            load_q6_chunk<LPR == 64>(W + row * row_bytes + (long)(c >> 2) * Q6K_BYTES, c, wk[n][i]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // token records: the clamped token t0 + min(t, nt - 1), so every record is valid
    q8pre_store<kQ6K>(pre, rec, XQ8, tok_bytes, t0, nt, nblk, total, nchunks);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);

    float acc[NR][TT];
#pragma unroll
    for (int n = 0; n < NR; n++)
#pragma unroll
        for (int t = 0; t < TT; t++) acc[n][t] = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const bool live = rl + i * LPR < nchunks;
        const int c = min(rl + i * LPR, nchunks - 1);
        const int h = (c >> 1) & 1, tq = c & 1;
#pragma unroll
        for (int n = 0; n < NR; n++) {
            const Q6Chunk& k6 = wk[n][i];
            const float d = h2f(k6.dbits);
            const uint32_t sa = h ? k6.sc[2] : k6.sc[0], sb = h ? k6.sc[3] : k6.sc[1];
            const int sA0 = (int8_t)(sa >> (16 * tq)), sA1 = (int8_t)(sa >> (16 * tq + 8));
            const int sB0 = (int8_t)(sb >> (16 * tq)), sB1 = (int8_t)(sb >> (16 * tq + 8));
            uint32_t qA[8], qB[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t l = k6.ql[k], hs = k6.qh[k] >> (2 * tq);
                qA[k] = (l & 0x0f0f0f0fu) | ((hs << 4) & 0x30303030u);
                qB[k] = ((l >> 4) & 0x0f0f0f0fu) | (hs & 0x30303030u);
            }
#pragma unroll
            for (int t = 0; t < TT; t++) {
                const uint4* r4 = reinterpret_cast<const uint4*>(rec + ((size_t)t * nchunks + c) * 20);
                const uint4 xa0 = r4[0], xa1 = r4[1], xb0 = r4[2], xb1 = r4[3], meta = r4[4];
                const float dxa = __uint_as_float(meta.x), dxb = __uint_as_float(meta.y);
                const int oA0 = -32 * (int)(int16_t)(meta.z & 0xffffu), oA1 = -32 * ((int)meta.z >> 16);
                const int oB0 = -32 * (int)(int16_t)(meta.w & 0xffffu), oB1 = -32 * ((int)meta.w >> 16);
                const uint32_t xa[8] = {xa0.x, xa0.y, xa0.z, xa0.w, xa1.x, xa1.y, xa1.z, xa1.w};
                const uint32_t xb[8] = {xb0.x, xb0.y, xb0.z, xb0.w, xb1.x, xb1.y, xb1.z, xb1.w};
                int iA0 = oA0, iA1 = oA1, iB0 = oB0, iB1 = oB1;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    iA0 = dot4((int)qA[k], (int)xa[k], iA0);
                    iB0 = dot4((int)qB[k], (int)xb[k], iB0);
                    iA1 = dot4((int)qA[k + 4], (int)xa[k + 4], iA1);
                    iB1 = dot4((int)qB[k + 4], (int)xb[k + 4], iB1);
                }
                float v = acc[n][t];
                v = fmaf((d * (float)sA0) * dxa, (float)iA0, v);
                v = fmaf((d * (float)sA1) * dxa, (float)iA1, v);
                v = fmaf((d * (float)sB0) * dxb, (float)iB0, v);
                v = fmaf((d * (float)sB1) * dxb, (float)iB1, v);
                acc[n][t] = live ? v : acc[n][t];
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const long row = row0 + (long)n * RPP;
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const float v = group_sum_last<LPR>(acc[n][t]);
            if (rl == LPR - 1 && row < rows && t < nt) Y[(size_t)(t0 + t) * rows + row] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------

static inline size_t qgemv_lds(int nb) { return (size_t)320 * nb + 4 * (16 + 256); }

template <int QT, int NT, int LPR, int CPL, int NR, int ACT, int EPI, bool PAIR, bool WL = false>
static hipError_t qgemv_cfg(const QGemvArgs& a, hipStream_t st) {
    constexpr int RW = (NT / 64) * (64 / LPR) * NR;
    const dim3 grid((unsigned)((a.rows0 + RW - 1) / RW));
    const size_t lds = qgemv_lds(a.nb) + (WL ? (size_t)RW * a.rb0 : 0);
    hipLaunchKernelGGL((k_qgemv<QT, NT, LPR, CPL, NR, ACT, EPI, PAIR, WL>), grid, dim3(NT), lds, st,
                       a);
    return hipGetLastError();
}

// the LDS-staged Q6_K rows: whole 16-byte rows, 16-byte aligned, in LDS
static bool q6k_wl_ok(const QGemvArgs& a, int rw) {
    return a.rb0 % 16 == 0 && (reinterpret_cast<uintptr_t>(a.W0) & 15) == 0 &&
           qgemv_lds(a.nb) + (size_t)rw * a.rb0 <= 64 * 1024;
}

template <int QT, int NT, int ACT, int EPI>
static hipError_t qgemv_pick(const QGemvArgs& a, hipStream_t st) {
    if constexpr (NT >= kWide) {
        if (pair_cfg(a.nb)) return qgemv_cfg<QT, NT, 32, 1, 1, ACT, EPI, true>(a, st);
        if constexpr (ACT == (int)QAct::Q8) return hipErrorInvalidValue;  // Q8 at 512: pairs only
    }
    KernCfg k = pick_cfg_nt(4 * a.nb, NT);
    if (a.shape & kShapeNR1) k.nr = 1;
#define AXF_Q(L, C, N) \
    if (k.lpr == L && k.cpl == C && k.nr == N)   \
        return qgemv_cfg<QT, NT, L, C, N, ACT, EPI, false>(a, st);
    if constexpr (ACT == (int)QAct::Q8 && NT == kWide) {
        // (pairs only, above)
    } else if constexpr (NT == kWider && ACT == (int)QAct::Norm) {
        AXF_GEMV_CFGS_1024_NORM(AXF_Q)
    } else if constexpr (NT == kWider) {
        AXF_GEMV_CFGS_1024(AXF_Q)
    } else if constexpr (NT == kWide && ACT == (int)QAct::Norm) {
        AXF_GEMV_CFGS_512_NORM(AXF_Q)
    } else if constexpr (NT == kWide) {
        AXF_GEMV_CFGS_512(AXF_Q)
    } else if constexpr (ACT == (int)QAct::F32) {
        AXF_GEMV_CFGS_GT4(AXF_Q)
    } else if constexpr (ACT == (int)QAct::Norm) {
        AXF_GEMV_CFGS_256_NORM(AXF_Q)
    } else {
        AXF_GEMV_CFGS(AXF_Q)
        AXF_GEMV_CFGS_256_NR1(AXF_Q)
    }
#undef AXF_Q
    return hipErrorInvalidValue;
}

bool qgemv_threads_ok(QAct act, int nb, int threads) {
    const int cpl = pick_cfg(4 * nb).cpl;
    switch (act) {
        case QAct::Q8: return threads == kThreads || (threads == kWide && pair_cfg(nb));
        case QAct::Norm: return nb <= 32 && (threads == kThreads || threads == kWide || threads == kWider);
        case QAct::F32:
            return threads == kWider ? cpl <= 3 : (threads == kWide ? cpl <= 4 : threads == kThreads && cpl > 4);
    }
    return false;
}

int qgemv_threads(QAct act, int nb) {
    if (act == QAct::Q8) return pair_cfg(nb) ? kWide : kThreads;
    if (act == QAct::Norm) return kWide;
    const int cpl = pick_cfg(4 * nb).cpl;
    return cpl <= 3 ? kWider : (cpl == 4 ? kWide : kThreads);
}

int qgemv_rows_per_wg(int nb, int threads, int shape) {
    if (threads >= kWide && pair_cfg(nb)) return (threads / 64) * 2;  // 32 lanes per row
    KernCfg k = pick_cfg_nt(4 * nb, threads);
    if (shape & kShapeNR1) k.nr = 1;
    return (threads / 64) * (64 / k.lpr) * k.nr;
}

// Instantiated: Q8 activations at 256 threads (the C-ABI GEMVs, residual
// projections); fused normalisation (K <= 8192, optionally with the SwiGLU
// epilogue) at 512 and 1024 threads; fp32 activations at 1024 (K <= 12288),
// 512 (K <= 16384) or 256 threads (qgemv_threads_ok).
hipError_t launch_qgemv(int qtype, QAct act, bool swiglu, QGemvArgs a, int threads,
                        hipStream_t st) {
    if (a.nb <= 0 || a.nb > kMaxBlocksPerRow || a.rows0 <= 0) return hipErrorInvalidValue;
    if (qtype != kQ4K && qtype != kQ6K) return hipErrorInvalidValue;
    if (!qgemv_threads_ok(act, a.nb, threads)) return hipErrorInvalidValue;
    const bool q4 = qtype == kQ4K;
    constexpr int Q8 = (int)QAct::Q8, NORM = (int)QAct::Norm, F32 = (int)QAct::F32;
#define AXF_QT(NT, ACT, EPI) \
    (q4 ? qgemv_pick<kQ4K, NT, ACT, EPI>(a, st) : qgemv_pick<kQ6K, NT, ACT, EPI>(a, st))
    if (swiglu) {
        if (act != QAct::Norm || threads < kWide ||
            a.rows0 % qgemv_rows_per_wg(a.nb, threads, a.shape) != 0)
            return hipErrorInvalidValue;
        return threads == kWider ? AXF_QT(kWider, NORM, EPI_SWIGLU) : AXF_QT(kWide, NORM, EPI_SWIGLU);
    }
    if (act == QAct::Q8)
        return threads == kWide ? AXF_QT(kWide, Q8, EPI_Y) : AXF_QT(kThreads, Q8, EPI_Y);
    if (act == QAct::Norm)
        return threads == kWider ? AXF_QT(kWider, NORM, EPI_Y)
                                 : (threads == kWide ? AXF_QT(kWide, NORM, EPI_Y) : AXF_QT(kThreads, NORM, EPI_Y));
    if (threads == kWider) return AXF_QT(kWider, F32, EPI_Y);
    if (threads == kWide) return AXF_QT(kWide, F32, EPI_Y);
    return AXF_QT(kThreads, F32, EPI_Y);
#undef AXF_QT
}

int qgemv_wgs(int rows, int nb, int threads, int shape) {
    const int rw = qgemv_rows_per_wg(nb, threads, shape);
    return (rows + rw - 1) / rw;
}

hipError_t launch_qgemv_argmax(int qtype, QGemvArgs a, int threads, hipStream_t st) {
    if (a.nb <= 0 || a.nb > 32 || a.rows0 <= 0 || !a.pv || !a.pi || a.accumulate ||
        (threads != kThreads && threads != kWide) || (qtype != kQ4K && qtype != kQ6K))
        return hipErrorInvalidValue;
    constexpr int NORM = (int)QAct::Norm;
    if (qtype == kQ4K)
        return threads == kWide ? qgemv_pick<kQ4K, kWide, NORM, EPI_ARGMAX>(a, st)
                                : qgemv_pick<kQ4K, kThreads, NORM, EPI_ARGMAX>(a, st);
    return threads == kWide ? qgemv_pick<kQ6K, kWide, NORM, EPI_ARGMAX>(a, st)
                            : qgemv_pick<kQ6K, kThreads, NORM, EPI_ARGMAX>(a, st);
}

template <int NT>
static hipError_t qgemv2_pick(QGemvArgs a, hipStream_t st) {
    const int rw = qgemv_rows_per_wg(a.nb, NT, a.shape);
    a.nwg0 = (a.rows0 + rw - 1) / rw;
    const dim3 grid((unsigned)(a.nwg0 + (a.rows1 + rw - 1) / rw));
    constexpr int NORM = (int)QAct::Norm;
    if (NT >= kWide && pair_cfg(a.nb)) {
        hipLaunchKernelGGL((k_qgemv2<NT, 32, 1, 1, NORM, true>), grid, dim3(NT), qgemv_lds(a.nb),
                           st, a);
        return hipGetLastError();
    }
    KernCfg k = pick_cfg_nt(4 * a.nb, NT);
    if (a.shape & kShapeNR1) k.nr = 1;
#define AXF_Q2(L, C, N)                                                                          \
    if (k.lpr == L && k.cpl == C && k.nr == N) {                                                 \
        hipLaunchKernelGGL((k_qgemv2<NT, L, C, N, NORM, false>), grid, dim3(NT), qgemv_lds(a.nb), \
                           st, a);                                                               \
        return hipGetLastError();                                                                \
    }
    if constexpr (NT == kWide) {
        AXF_GEMV_CFGS_512_NORM(AXF_Q2)
    } else {
        AXF_GEMV_CFGS_256_NORM(AXF_Q2)
    }
#undef AXF_Q2
    return hipErrorInvalidValue;
}

hipError_t launch_qgemv2(QAct act, QGemvArgs a, int threads, hipStream_t st) {
    if (act != QAct::Norm || (threads != kWide && threads != kThreads) || a.nb <= 0 || a.nb > 32 ||
        a.rows0 <= 0 || a.rows1 <= 0)
        return hipErrorInvalidValue;
    return threads == kWide ? qgemv2_pick<kWide>(a, st) : qgemv2_pick<kThreads>(a, st);
}

// Q4_K x F32 GEMV workgroup: 512 threads (config 1, 4096x4096: 5.37 us at 256
// threads, 5.20 at 512, 5.21 at 1024)
constexpr int kF32Threads = 512;

template <int LPR, int CPL, int NR>
static hipError_t launch_cfg(GemvKind kind, float* y, const void* W, const void* x, int rows,
                             int nb, long row_bytes, int accumulate, hipStream_t st) {
    constexpr int rows_per_wg = kWaves * (64 / LPR) * NR;
    const dim3 grid((unsigned)((rows + rows_per_wg - 1) / rows_per_wg));
    const dim3 block(kThreads);
    const auto* Wb = static_cast<const uint8_t*>(W);
    if (kind == GemvKind::Q4K_Q8 || kind == GemvKind::Q6K_Q8) {
        QGemvArgs a{};
        a.W0 = Wb;
        a.rb0 = row_bytes;
        a.rows0 = rows;
        a.y0 = y;
        a.nb = nb;
        a.accumulate = accumulate;
        a.xq8 = static_cast<const uint8_t*>(x);
        if (pair_cfg(nb))  // half-block units, 512 threads
            return kind == GemvKind::Q4K_Q8
                       ? qgemv_cfg<kQ4K, kWide, 32, 1, 1, (int)QAct::Q8, EPI_Y, true>(a, st)
                       : qgemv_cfg<kQ6K, kWide, 32, 1, 1, (int)QAct::Q8, EPI_Y, true>(a, st);
        // half-block units of 16 lanes, 512 threads (5-8 super-blocks per row):
        // the 151936 x 2048 Q6_K head 54.9 -> 47.4 us against one chunk per lane
        // with aligned dwords (two rows per lane group 51.9 us, 256 threads 48.5 us).
        // Q6_K rows of a multiple of 16 bytes (8 super-blocks) staged in LDS
        // per wave, 256 threads (five workgroups per CU): 48.1 -> 44.4 us (512
        // threads, two per CU: 49.5 us; 128 threads: 46.6-47.4 us)
        if (nb >= 5 && nb <= 8)
            return kind == GemvKind::Q4K_Q8
                       ? qgemv_cfg<kQ4K, kWide, 16, 1, 1, (int)QAct::Q8, EPI_Y, true>(a, st)
                   : q6k_wl_ok(a, 16)
                       ? qgemv_cfg<kQ6K, kThreads, 16, 1, 1, (int)QAct::Q8, EPI_Y, true, true>(a, st)
                       : qgemv_cfg<kQ6K, kWide, 16, 1, 1, (int)QAct::Q8, EPI_Y, true>(a, st);
        return kind == GemvKind::Q4K_Q8
                   ? qgemv_cfg<kQ4K, kThreads, LPR, CPL, NR, (int)QAct::Q8, EPI_Y, false>(a, st)
                   : qgemv_cfg<kQ6K, kThreads, LPR, CPL, NR, (int)QAct::Q8, EPI_Y, false>(a, st);
    }
    if (kind == GemvKind::Q4K_F32) {
        constexpr int NT = kF32Threads;
        constexpr int RW = (NT / 64) * (64 / LPR) * NR;
        const dim3 g2((unsigned)((rows + RW - 1) / RW));
        hipLaunchKernelGGL((k_gemv_q4k_f32<LPR, CPL, NR, NT>), g2, dim3(NT),
                           (size_t)nb * QK_K * 4 * 17 / 16, st, y, Wb,
                           static_cast<const float*>(x), rows, nb, row_bytes, accumulate);
    } else
        hipLaunchKernelGGL((k_gemv_q6k_f32<LPR, CPL, NR>), grid, block,
                           (size_t)nb * QK_K * 4 * 9 / 8, st, y, Wb,
                           static_cast<const float*>(x), rows, nb, row_bytes, accumulate);
    return hipGetLastError();
}

// Largest K handled: 8 chunks per lane at 64 lanes -> kMaxBlocksPerRow = 128 super-blocks.
hipError_t launch_gemv(GemvKind kind, float* y, const void* W, const void* x, int rows, int nb,
                       long row_bytes, int accumulate, hipStream_t st) {
    const KernCfg k = pick_cfg(4 * nb);
#define AXF_GEMV_CASE(L, C, N) \
    if (k.lpr == L && k.cpl == C && k.nr == N)                                                \
        return launch_cfg<L, C, N>(kind, y, W, x, rows, nb, row_bytes, accumulate, st);
    AXF_GEMV_CFGS(AXF_GEMV_CASE)
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
    AXF_GEMV_CFGS(AXF_GEMM_CASE)
#undef AXF_GEMM_CASE
    return hipErrorInvalidValue;
}

static hipError_t launch_gemm_dot4(float* Y, const void* W, const void* XQ8, int rows, int T,
                                   int nb, long row_bytes, hipStream_t st) {
    // token tile: as many tokens as fit 64 KiB of LDS records (80 B per chunk)
    const size_t per_tok = (size_t)4 * nb * 80;
    int tt = (int)(65536 / per_tok);
    if (T >= 8 && tt >= 8) return launch_gemm_tt<8>(Y, W, XQ8, rows, T, nb, row_bytes, st);
    if (T >= 4 && tt >= 4) return launch_gemm_tt<4>(Y, W, XQ8, rows, T, nb, row_bytes, st);
    if (T >= 2 && tt >= 2) return launch_gemm_tt<2>(Y, W, XQ8, rows, T, nb, row_bytes, st);
    return launch_gemm_tt<1>(Y, W, XQ8, rows, T, nb, row_bytes, st);
}

template <int LPR, int CPL, int NR, int TT>
static hipError_t launch_gemm6_cfg(float* Y, const void* W, const void* XQ8, int rows, int T,
                                   int nb, long row_bytes, hipStream_t st) {
    constexpr int rows_per_wg = kWaves * (64 / LPR) * NR;
    const dim3 grid((unsigned)((rows + rows_per_wg - 1) / rows_per_wg));
    const size_t lds = (size_t)TT * 4 * nb * 80;
    for (int t0 = 0; t0 < T; t0 += TT) {
        const int nt = T - t0 < TT ? T - t0 : TT;
        hipLaunchKernelGGL((k_gemm_q6k_q8<LPR, CPL, NR, TT>), grid, dim3(kThreads), lds, st, Y,
                           static_cast<const uint8_t*>(W), static_cast<const uint8_t*>(XQ8), rows,
                           nb, row_bytes, t0, nt);
    }
    return hipGetLastError();
}

template <int TT>
static hipError_t launch_gemm6_tt(float* Y, const void* W, const void* XQ8, int rows, int T,
                                  int nb, long row_bytes, hipStream_t st) {
    const KernCfg k = pick_cfg(4 * nb);
#define AXF_GEMM6_CASE(L, C, N)                                                            \
    if (k.lpr == L && k.cpl == C && k.nr == N)                                             \
        return launch_gemm6_cfg<L, C, N, TT>(Y, W, XQ8, rows, T, nb, row_bytes, st);
    AXF_GEMV_CFGS(AXF_GEMM6_CASE)
#undef AXF_GEMM6_CASE
    return hipErrorInvalidValue;
}

static hipError_t launch_gemm6_dot4(float* Y, const void* W, const void* XQ8, int rows, int T,
                                    int nb, long row_bytes, hipStream_t st) {
    // token tile: as many tokens as fit 64 KiB of LDS records (80 B per chunk),
    // and few enough that the decoded chunks and accumulators stay in VGPRs
    const size_t per_tok = (size_t)4 * nb * 80;
    int tt = (int)(65536 / per_tok);
    const int cpl = pick_cfg(4 * nb).cpl;
    if (cpl > 3 && tt > 4) tt = 4;
    if (cpl > 6 && tt > 2) tt = 2;
    if (T >= 8 && tt >= 8) return launch_gemm6_tt<8>(Y, W, XQ8, rows, T, nb, row_bytes, st);
    if (T >= 4 && tt >= 4) return launch_gemm6_tt<4>(Y, W, XQ8, rows, T, nb, row_bytes, st);
    if (T >= 2 && tt >= 2) return launch_gemm6_tt<2>(Y, W, XQ8, rows, T, nb, row_bytes, st);
    return launch_gemm6_tt<1>(Y, W, XQ8, rows, T, nb, row_bytes, st);
}

GemmPath gemm_resolve(GemmPath path, int T) {
    if (path != GemmPath::Auto) return path;
    if (T < kGemmMfmaMinT) return GemmPath::Dot4;
    return T <= kGemmStreamMaxT ? GemmPath::Stream : GemmPath::Mfma;
}

size_t gemm_scratch_bytes(int qtype, GemmPath path, int T, int nb, int rows) {
    const GemmPath p = gemm_resolve(path, T);
    if (p == GemmPath::Dot4) return 0;
    if (qtype == AXF_TYPE_Q6_K) return gemm_mfma_q6k_scratch_bytes(T, nb);
    const size_t mf = gemm_mfma_scratch_bytes(T, nb);
    if (p == GemmPath::Stream && gemm_stream_q4k_ok(T, nb, rows)) {
        // room for the Mfma fallback (unaligned operands) as well
        const size_t sb = gemm_stream_scratch_bytes(T, nb, rows);
        return sb > mf ? sb : mf;
    }
    return mf;
}

hipError_t launch_gemm_q4k_q8(float* Y, const void* W, const void* XQ8, int rows, int T, int nb,
                              long row_bytes, GemmPath path, void* scratch, hipStream_t st) {
    const GemmPath p = gemm_resolve(path, T);
    if (p == GemmPath::Stream && gemm_stream_q4k_ok(T, nb, rows) &&
        (((uintptr_t)W | (uintptr_t)XQ8 | (uintptr_t)row_bytes) & 15) == 0)
        return launch_gemm_stream_q4k_q8(Y, W, XQ8, rows, T, nb, row_bytes, scratch, st);
    if (p != GemmPath::Dot4)
        return launch_gemm_mfma_q4k_q8(Y, W, XQ8, rows, T, nb, row_bytes, scratch, st);
    return launch_gemm_dot4(Y, W, XQ8, rows, T, nb, row_bytes, st);
}

hipError_t launch_gemm_q6k_q8(float* Y, const void* W, const void* XQ8, int rows, int T, int nb,
                              long row_bytes, GemmPath path, void* scratch, hipStream_t st) {
    // the matrix-core kernel copies 16-byte-aligned spans of the 2-byte-aligned
    // blocks: it needs a last block that ends on a 16-byte boundary (and < 2 GiB)
    if (gemm_resolve(path, T) != GemmPath::Dot4 && gemm_mfma_q6k_ok(W, rows, nb, row_bytes))
        return launch_gemm_mfma_q6k_q8(Y, W, XQ8, rows, T, nb, row_bytes, scratch, st);
    return launch_gemm6_dot4(Y, W, XQ8, rows, T, nb, row_bytes, st);
}

}  // namespace axf
