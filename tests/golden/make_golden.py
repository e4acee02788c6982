"""Write tests/golden/ref_kernels.npz: input/output vectors of the reference's
own x86 kernels, compiled from their sources into oracle/_ref/libaxf_ref.so by
oracle/Makefile (no reference source is copied; only data is stored).

    make -C oracle && python tests/golden/make_golden.py

Inputs are drawn with numpy's PCG64 from fixed seeds, independent of the
package's synthetic-weight generator.  Every array is plain numeric data
(np.load(..., allow_pickle=False) reads it).

Reference functions exercised (src/backend/cpu_x86/kernels/):
  gemv_q4k_avx2_range        gemv_q4k_avx2.cpp:72-238     Q4_K x f32
  gemv_q6k_avx2_range        gemv_q6k_avx2.cpp:85-244     Q6_K x f32
  quantize_q8_avx2           quant_q8_avx2.cpp:33-84      f32 -> Q8_0
  gemv_q4k_q8_{avx2,avxvnni}_range                        Q4_K x Q8_0, 4-row tiles
  repack_q4k_8rows           gemv_q4k_r8_avx2.cpp:102-136 r8 layout
  gemv_q4k_r8_{avx2,avxvnni}_range                        Q4_K(r8) x Q8_0 (decode kernel)
  gemv_q6k_q8_avx2_range     gemv_q6k_q8_avx2.cpp:104-205 Q6_K x Q8_0
  gemm_q4k_q8_{avx2,avxvnni}_range                        Q4_K x Q8_0, T tokens

Dequantisation has no separately buildable reference entry (the scalar
dequant lives in llama_model.cpp, which needs a CMake-generated header), so the
golden dequantised matrices are read out of gemv_*_avx2_range with one-hot
activations: y_r = sum_k w_rk x_k with x = e_j is exactly w_rj (the other
products are zeros, and the one non-zero product is exact), which is the
fused (d*sc)*q - dmin*m of the reference's kernels.
"""
from __future__ import annotations

import ctypes as C
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent / "ref_kernels.npz"
Q4K, Q6K = O.Q4K, O.Q6K


def p(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


def blocks(qtype: int, n: int, rng: np.random.Generator, realistic: bool) -> np.ndarray:
    """n blocks of random bytes with finite fp16 scales.  realistic: scales in
    [1e-4, 1e-2] like trained weights; else any finite fp16 (zero and
    subnormal included)."""
    bb = O.BLOCK_BYTES[qtype]
    blk = rng.integers(0, 256, size=(n, bb), dtype=np.uint8)
    if realistic:
        h = rng.uniform(1e-4, 1e-2, size=(n, 2)).astype(np.float16).view(np.uint16)
    else:
        h = rng.integers(0, 0x7C00, size=(n, 2), dtype=np.uint16)
        h |= rng.integers(0, 2, size=(n, 2), dtype=np.uint16) << 15
        h[0] = 0
        h[1] = 0x0001  # smallest subnormal
    hb = np.ascontiguousarray(h).view(np.uint8).reshape(n, 4)
    if qtype == Q4K:
        blk[:, 0:4] = hb
    else:
        blk[:, 208:210] = hb[:, 0:2]
    return blk.reshape(-1)


def acts(n: int, rng: np.random.Generator) -> np.ndarray:
    x = rng.standard_normal(n).astype(np.float32)
    x *= rng.choice(np.array([1e-3, 1.0, 30.0], np.float32), n)
    return x


def edge_acts() -> np.ndarray:
    """Q8_0 edge blocks: zeros, exact .5 ties, an outlier, tiny values, negatives."""
    x = np.zeros(256, np.float32)
    x[32:64] = np.arange(-15.5, 16.5, 1.0, dtype=np.float32)
    x[63] = 127.0                       # amax 127 -> id == 1, ties stay ties
    x[64:96] = 1e-3
    x[64] = 1e6
    x[96:128] = -np.linspace(0.0, 2.0, 32, dtype=np.float32)
    x[128:160] = 1e-30
    x[160:192] = np.float32(63.5)       # all equal: every value maps to 127
    x[192:256] = np.linspace(-1, 1, 64, dtype=np.float32) ** 3
    return x


def onehot_dequant(fn, W: np.ndarray, rows: int, cols: int, rb: int) -> np.ndarray:
    D = np.empty((rows, cols), np.float32)
    e = np.zeros(cols, np.float32)
    y = np.empty(rows, np.float32)
    for j in range(cols):
        e[:] = 0.0
        e[j] = 1.0
        fn(p(y), p(W), p(e), 0, rows, cols, rb)
        D[:, j] = y
    return D


def main() -> None:
    R = O.ref
    if R is None:
        raise SystemExit("oracle/_ref/libaxf_ref.so missing: run `make -C oracle` where "
                         "/root/reference exists")
    rng = np.random.default_rng(20240611)
    rows, cols, T = 16, 512, 4
    out: dict[str, np.ndarray] = {}
    vnni = bool(R.ref_has_avxvnni())
    out["has_vnni"] = np.array([int(vnni)], np.int32)
    out["shape"] = np.array([rows, cols, T], np.int32)

    x = acts(cols, rng)
    X = np.stack([acts(cols, rng) for _ in range(T)])
    out["x"] = x
    out["X"] = X
    xq8 = np.empty(cols // 32 * 36, np.uint8)
    R.ref_quantize_q8_0(p(xq8), p(x), cols)
    out["xq8"] = xq8
    XQ8 = np.empty(T * cols // 32 * 36, np.uint8)
    R.ref_quantize_q8_0(p(XQ8), p(X), T * cols)
    out["XQ8"] = XQ8
    xe = edge_acts()
    xeq8 = np.empty(256 // 32 * 36, np.uint8)
    R.ref_quantize_q8_0(p(xeq8), p(xe), 256)
    out["x_edge"] = xe
    out["x_edge_q8"] = xeq8

    for tag, realistic in (("", True), ("r", False)):
        for qt, name in ((Q4K, "q4"), (Q6K, "q6")):
            rb = O.row_bytes(qt, cols)
            W = blocks(qt, rows * cols // 256, rng, realistic)
            key = name + tag
            out[f"W_{key}"] = W
            f32 = R.ref_gemv_q4k_f32 if qt == Q4K else R.ref_gemv_q6k_f32
            out[f"deq_{key}"] = onehot_dequant(f32, W, rows, cols, rb)
            y = np.empty(rows, np.float32)
            f32(p(y), p(W), p(x), 0, rows, cols, rb)
            out[f"y_f32_{key}"] = y.copy()
            if qt == Q4K:
                R.ref_gemv_q4k_q8(p(y), p(W), p(xq8), 0, rows, cols, rb, 0)
                out[f"y_q8_avx2_{key}"] = y.copy()
                if vnni:
                    R.ref_gemv_q4k_q8(p(y), p(W), p(xq8), 0, rows, cols, rb, 1)
                    out[f"y_q8_vnni_{key}"] = y.copy()
                r8 = np.empty_like(W)
                R.ref_repack_q4k_r8(p(r8), p(W), rows, cols)
                out[f"r8_{key}"] = r8
                R.ref_gemv_q4k_r8(p(y), p(r8), p(xq8), 0, rows, cols, 0)
                out[f"y_r8_avx2_{key}"] = y.copy()
                if vnni:
                    R.ref_gemv_q4k_r8(p(y), p(r8), p(xq8), 0, rows, cols, 1)
                    out[f"y_r8_vnni_{key}"] = y.copy()
                Y = np.empty(T * rows, np.float32)
                R.ref_gemm_q4k_q8(p(Y), p(W), p(XQ8), rows, T, cols, rb, 0, rows, 0)
                out[f"Y_gemm_avx2_{key}"] = Y.reshape(T, rows).copy()
                if vnni:
                    R.ref_gemm_q4k_q8(p(Y), p(W), p(XQ8), rows, T, cols, rb, 0, rows, 1)
                    out[f"Y_gemm_vnni_{key}"] = Y.reshape(T, rows).copy()
            else:
                R.ref_gemv_q6k_q8(p(y), p(W), p(xq8), 0, rows, cols, rb)
                out[f"y_q8_{key}"] = y.copy()
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays, vnni={vnni})")


if __name__ == "__main__":
    main()
