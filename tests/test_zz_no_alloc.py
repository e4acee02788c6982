"""axf_hip_gemm_q4k_q8_noalloc: the Q4_K x Q8_0 GEMM without device allocation
(its scratch is a fixed device array inside the library).  Through the C-ABI
it must return the bits of axf_hip_gemm_q4k_q8 (same kernels, same inputs):
two calls in a row, the second with fewer tokens, on the matrix-core paths
(which use the scratch) and on the dot4 path (which does not); where the
automatic kernel's split-K partials exceed the fixed array the LDS-ring kernel
runs (the bits of path 2); sizes whose scratch exceeds the array on every
path are refused with an error."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def test_noalloc_gemm_matches_allocating_gemm(ctx):
    from llm_core_amd import _ffi, hip

    fn = _ffi.lib.axf_hip_gemm_q4k_q8_noalloc
    rows, cols = 2816, 4096
    rb = hip.row_bytes(hip.AXF_TYPE_Q4_K, cols)
    W = hip.synth_weight(hip.AXF_TYPE_Q4_K, rows, cols, 61)
    dW = ctx.upload(W)
    for T in (64, 16, 3):          # 64 and 16: matrix cores, split-K partials; 3: dot4
        X = hip.synth_normal(T * cols, 62 + T)
        XQ8 = np.concatenate([O.quantize_q8_0(X[t * cols:(t + 1) * cols]) for t in range(T)])
        dX = ctx.upload(XQ8)
        nan = np.full(T * rows, np.nan, np.float32)
        dA, dB = ctx.upload(nan), ctx.upload(nan)
        ctx.gemm_q4k_q8(dA, dW, dX, rows, T, cols, rb)
        rc = fn(ctx.handle, C.c_void_p(int(dB)), C.c_void_p(int(dW)), C.c_void_p(int(dX)), rows,
                T, cols, rb)
        assert rc == 0, _ffi.last_error()
        a = ctx.download(dA, np.float32, T * rows)
        b = ctx.download(dB, np.float32, T * rows)
        print(f"  T={T}: noalloc vs allocating GEMM bit-exact: {np.array_equal(a, b)}", flush=True)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        # and both against the oracle's GEMM (gemm_q4k_q8_avx2_range) at the north-star bound
        want = O.gemm_q4k_q8(W, XQ8, rows, T, cols).reshape(-1)
        assert np.all(np.abs(b - want) <= 1e-4 + 1e-3 * np.abs(want))


def test_noalloc_gemm_falls_back_to_the_ring_kernel(ctx):
    from llm_core_amd import _ffi, hip

    fn = _ffi.lib.axf_hip_gemm_q4k_q8_noalloc
    rows, cols, T = 11008, 4096, 64   # split-K partials: 4 x 64 x 11008 x 4 B > 8 MiB
    rb = hip.row_bytes(hip.AXF_TYPE_Q4_K, cols)
    W = hip.synth_weight(hip.AXF_TYPE_Q4_K, rows, cols, 71)
    dW = ctx.upload(W)
    X = hip.synth_normal(T * cols, 72)
    XQ8 = np.concatenate([O.quantize_q8_0(X[t * cols:(t + 1) * cols]) for t in range(T)])
    dX = ctx.upload(XQ8)
    nan = np.full(T * rows, np.nan, np.float32)
    dA, dB = ctx.upload(nan), ctx.upload(nan)
    ctx.gemm_q4k_q8(dA, dW, dX, rows, T, cols, rb, path=2)
    rc = fn(ctx.handle, C.c_void_p(int(dB)), C.c_void_p(int(dW)), C.c_void_p(int(dX)), rows, T,
            cols, rb)
    assert rc == 0, _ffi.last_error()
    a = ctx.download(dA, np.float32, T * rows)
    b = ctx.download(dB, np.float32, T * rows)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_noalloc_gemm_refuses_oversized_scratch(ctx):
    from llm_core_amd import _ffi, hip

    fn = _ffi.lib.axf_hip_gemm_q4k_q8_noalloc
    rows, cols, T = 256, 11008, 352        # needs 8.7 MB of re-layout, above 8 MiB
    rb = hip.row_bytes(hip.AXF_TYPE_Q4_K, cols)
    dW = ctx.alloc(rows * rb)
    dX = ctx.alloc(T * cols // 32 * 36)
    dY = ctx.alloc(T * rows * 4)
    rc = fn(ctx.handle, C.c_void_p(int(dY)), C.c_void_p(int(dW)), C.c_void_p(int(dX)), rows, T,
            cols, rb)
    assert rc == _ffi.AXF_ERR_INVALID_ARG
    assert "scratch" in _ffi.last_error()
    # 320 tokens (8.0 MB of re-layout) still fit: all-zero weights give zeros
    T = 320
    dW = ctx.upload(np.zeros(rows * rb, np.uint8))
    dX = ctx.upload(np.zeros(T * cols // 32 * 36, np.uint8))
    dY = ctx.upload(np.full(T * rows, np.nan, np.float32))
    rc = fn(ctx.handle, C.c_void_p(int(dY)), C.c_void_p(int(dW)), C.c_void_p(int(dX)), rows, T,
            cols, rb)
    assert rc == 0, _ffi.last_error()
    assert not np.any(ctx.download(dY, np.float32, T * rows))
