"""Thin Python handle over the C-ABI for tests and benchmarks.

Device memory is allocated through the library itself (axf_hip_alloc); numpy
arrays are copied in and out with the blocking copies of the C-ABI.  All
compute goes through libaxf_hip.so.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _ffi
from ._ffi import AXF_TYPE_Q4_K, AXF_TYPE_Q6_K, call, lib

Q8_0_BYTES = 36


def device_count() -> int:
    n = C.c_int(0)
    call("axf_hip_device_count", C.byref(n))
    return n.value


def row_bytes(qtype: int, cols: int) -> int:
    return int(lib.axf_row_bytes(qtype, cols))


class Buffer:
    """Owned device allocation."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        call("axf_hip_alloc", ctx.handle, C.c_size_t(self.nbytes), C.byref(p))
        self.ptr = p.value or 0

    def free(self) -> None:
        if self.ptr:
            call("axf_hip_free", self.ctx.handle, C.c_void_p(self.ptr))
            self.ptr = 0

    def at(self, offset: int) -> int:
        return self.ptr + int(offset)

    def __int__(self) -> int:
        return self.ptr


class Context:
    def __init__(self, device: int = 0):
        h = C.c_void_p()
        call("axf_hip_create", device, C.byref(h))
        self.handle = h
        self._bufs: list[Buffer] = []

    # ---- lifecycle / memory ---------------------------------------------
    def close(self) -> None:
        if self.handle:
            for b in self._bufs:
                b.free()
            self._bufs.clear()
            call("axf_hip_destroy", self.handle)
            self.handle = None

    def __enter__(self) -> "Context":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def device_name(self) -> str:
        buf = C.create_string_buffer(256)
        call("axf_hip_device_name", self.handle, buf, 256)
        return buf.value.decode()

    def alloc(self, nbytes: int) -> Buffer:
        b = Buffer(self, max(int(nbytes), 16))
        self._bufs.append(b)
        return b

    def upload(self, arr: np.ndarray) -> Buffer:
        a = np.ascontiguousarray(arr)
        b = self.alloc(a.nbytes)
        call("axf_hip_memcpy_h2d", self.handle, C.c_void_p(b.ptr), a.ctypes.data_as(C.c_void_p),
             C.c_size_t(a.nbytes))
        return b

    def write(self, dst: int, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr)
        call("axf_hip_memcpy_h2d", self.handle, C.c_void_p(int(dst)), a.ctypes.data_as(C.c_void_p),
             C.c_size_t(a.nbytes))

    def copy(self, dst: int, src: int, nbytes: int) -> None:
        """Device-to-device copy, asynchronous on the context stream."""
        call("axf_hip_memcpy_d2d", self.handle, C.c_void_p(int(dst)), C.c_void_p(int(src)),
             C.c_size_t(int(nbytes)))

    def download(self, src: int, dtype, count: int) -> np.ndarray:
        out = np.empty(int(count), dtype=dtype)
        call("axf_hip_memcpy_d2h", self.handle, out.ctypes.data_as(C.c_void_p), C.c_void_p(int(src)),
             C.c_size_t(out.nbytes))
        return out

    def sync(self) -> None:
        call("axf_hip_sync", self.handle)

    # ---- kernels -----------------------------------------------------------
    def dequant(self, qtype: int, y: int, W: int, n_blocks: int) -> None:
        name = "axf_hip_dequant_q4k" if qtype == AXF_TYPE_Q4_K else "axf_hip_dequant_q6k"
        call(name, self.handle, C.c_void_p(int(y)), C.c_void_p(int(W)), C.c_int64(n_blocks))

    def quantize_q8_0(self, yq8: int, x: int, n: int) -> None:
        call("axf_hip_quantize_q8_0", self.handle, C.c_void_p(int(yq8)), C.c_void_p(int(x)), n)

    def gemv_f32(self, qtype: int, y: int, W: int, x: int, rows: int, cols: int, rb: int) -> None:
        name = "axf_hip_gemv_q4k_f32" if qtype == AXF_TYPE_Q4_K else "axf_hip_gemv_q6k_f32"
        call(name, self.handle, C.c_void_p(int(y)), C.c_void_p(int(W)), C.c_void_p(int(x)), rows,
             cols, C.c_size_t(rb))

    def gemv_q8(self, qtype: int, y: int, W: int, xq8: int, rows: int, cols: int, rb: int,
                accumulate: bool = False) -> None:
        name = "axf_hip_gemv_q4k_q8" if qtype == AXF_TYPE_Q4_K else "axf_hip_gemv_q6k_q8"
        call(name, self.handle, C.c_void_p(int(y)), C.c_void_p(int(W)), C.c_void_p(int(xq8)),
             rows, cols, C.c_size_t(rb), 1 if accumulate else 0)

    def gemm_q4k_q8(self, Y: int, W: int, XQ8: int, rows: int, T: int, cols: int, rb: int,
                    path: int | None = None) -> None:
        """Token-major Q4_K x Q8_0 GEMM; path None = automatic, 1 dot4, 2 matrix cores
        (LDS ring), 3 matrix cores with the weights streamed into registers."""
        if path is None:
            call("axf_hip_gemm_q4k_q8", self.handle, C.c_void_p(int(Y)), C.c_void_p(int(W)),
                 C.c_void_p(int(XQ8)), rows, T, cols, C.c_size_t(rb))
        else:
            call("axf_hip_gemm_q4k_q8_path", self.handle, C.c_void_p(int(Y)), C.c_void_p(int(W)),
                 C.c_void_p(int(XQ8)), rows, T, cols, C.c_size_t(rb), int(path))

    def gemm_q6k_q8(self, Y: int, W: int, XQ8: int, rows: int, T: int, cols: int, rb: int,
                    path: int | None = None) -> None:
        """Token-major Q6_K x Q8_0 GEMM; path None = automatic, 1 dot4, 2 matrix cores."""
        if path is None:
            call("axf_hip_gemm_q6k_q8", self.handle, C.c_void_p(int(Y)), C.c_void_p(int(W)),
                 C.c_void_p(int(XQ8)), rows, T, cols, C.c_size_t(rb))
        else:
            call("axf_hip_gemm_q6k_q8_path", self.handle, C.c_void_p(int(Y)), C.c_void_p(int(W)),
                 C.c_void_p(int(XQ8)), rows, T, cols, C.c_size_t(rb), int(path))

    def sample(self, logits: int, n_vocab: int, temperature: float = 1.0, top_k: int = 40,
               top_p: float = 1.0, rep_penalty: float = 1.0, rep_penalty_last_n: int = 64,
               hist=(), r: float = 0.0) -> int:
        """One token choice (axf_hip_sample); the penalty is applied to the device
        logits in place."""
        s = sampling(temperature, top_k, top_p, rep_penalty, rep_penalty_last_n)
        h = np.ascontiguousarray(hist, np.int32)
        tok = C.c_int32()
        call("axf_hip_sample", self.handle, C.c_void_p(int(logits)), n_vocab, C.byref(s),
             h.ctypes.data_as(C.c_void_p) if h.size else None, int(h.size), float(r),
             C.byref(tok))
        return int(tok.value)

    def argmax(self, idx: int, x: int, n: int) -> None:
        call("axf_hip_argmax_f32", self.handle, C.c_void_p(int(idx)), C.c_void_p(int(x)), n)

    def rmsnorm(self, y: int | None, yq8: int | None, x: int, w: int, n: int, eps: float) -> None:
        call("axf_hip_rmsnorm", self.handle, C.c_void_p(int(y) if y else None),
             C.c_void_p(int(yq8) if yq8 else None), C.c_void_p(int(x)), C.c_void_p(int(w)), n,
             C.c_float(eps))

    def rope(self, dst: int, src: int, pos: int, n_heads: int, hd: int, cos_t: int,
             sin_t: int) -> None:
        call("axf_hip_rope", self.handle, C.c_void_p(int(dst)), C.c_void_p(int(src)), pos, n_heads,
             hd, C.c_void_p(int(cos_t)), C.c_void_p(int(sin_t)))

    def attn_decode(self, out: int, outq8: int | None, q: int, k: int, v: int, seq: int,
                    n_heads: int, n_kv_heads: int, hd: int) -> None:
        call("axf_hip_attn_decode", self.handle, C.c_void_p(int(out)),
             C.c_void_p(int(outq8) if outq8 else None), C.c_void_p(int(q)), C.c_void_p(int(k)),
             C.c_void_p(int(v)), seq, n_heads, n_kv_heads, hd)

    def swiglu(self, out: int | None, outq8: int | None, gate: int, up: int, n: int) -> None:
        call("axf_hip_swiglu", self.handle, C.c_void_p(int(out) if out else None),
             C.c_void_p(int(outq8) if outq8 else None), C.c_void_p(int(gate)), C.c_void_p(int(up)), n)

    def add(self, y: int, a: int, b: int, n: int) -> None:
        call("axf_hip_add", self.handle, C.c_void_p(int(y)), C.c_void_p(int(a)), C.c_void_p(int(b)), n)

    def embed(self, out: int, qtype: int, W: int, token: int, rows: int, cols: int) -> None:
        call("axf_hip_embed", self.handle, C.c_void_p(int(out)), qtype, C.c_void_p(int(W)), token,
             rows, cols)

    def bench_read(self, bufs, nbytes: int, unroll: int, wgs: int, reps: int) -> float:
        """Milliseconds for reps passes of a plain streaming read over bufs."""
        arr = (C.c_void_p * len(bufs))(*[int(b) for b in bufs])
        ms = C.c_float(0)
        call("axf_hip_bench_read", self.handle, arr, len(bufs), C.c_size_t(nbytes), unroll, wgs,
             reps, C.byref(ms))
        return ms.value

    def bench_set_eager(self, eager: bool) -> None:
        """Benchmark helpers launch directly instead of replaying captured graphs."""
        call("axf_hip_bench_set_eager", self.handle, 1 if eager else 0)

    def timer_start(self) -> None:
        call("axf_hip_timer_start", self.handle)

    def timer_stop(self) -> float:
        ms = C.c_float(0)
        call("axf_hip_timer_stop", self.handle, C.byref(ms))
        return ms.value

    def bench_gemv(self, kind: int, y: int, W_list, x: int, rows: int, cols: int, rb: int,
                   reps: int) -> float:
        """Milliseconds for reps*len(W_list) graph-replayed GEMV launches
        (kind 0 Q4_K x Q8_0, 1 Q6_K x Q8_0, 2 Q4_K x F32, 3 Q6_K x F32)."""
        arr = (C.c_void_p * len(W_list))(*[int(w) for w in W_list])
        ms = C.c_float(0)
        call("axf_hip_bench_gemv", self.handle, kind, C.c_void_p(int(y)), arr, len(W_list),
             C.c_void_p(int(x)), rows, cols, C.c_size_t(rb), reps, C.byref(ms))
        return ms.value

    def bench_gemm(self, Y: int, W_list, XQ8: int, rows: int, T: int, cols: int, rb: int,
                   reps: int, path: int = 0, qtype: int = AXF_TYPE_Q4_K) -> float:
        """Milliseconds for reps*len(W_list) graph-replayed Q4_K (or Q6_K) x Q8_0
        GEMM launches of T tokens (path 0 automatic, 1 dot4, 2 matrix cores)."""
        arr = (C.c_void_p * len(W_list))(*[int(w) for w in W_list])
        ms = C.c_float(0)
        call("axf_hip_bench_gemm", self.handle, int(qtype), C.c_void_p(int(Y)), arr, len(W_list),
             C.c_void_p(int(XQ8)), rows, T, cols, C.c_size_t(rb), int(path), reps, C.byref(ms))
        return ms.value


def rope_table(head_dim: int, theta: float, max_pos: int) -> tuple[np.ndarray, np.ndarray]:
    c = np.empty(max_pos * (head_dim // 2), np.float32)
    s = np.empty_like(c)
    call("axf_rope_table", c.ctypes.data_as(C.c_void_p), s.ctypes.data_as(C.c_void_p), head_dim,
         C.c_float(theta), max_pos)
    return c, s


def synth_normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(int(n), np.float32)
    call("axf_synth_normal", out.ctypes.data_as(C.c_void_p), C.c_int64(out.size), C.c_uint64(seed),
         C.c_float(mean), C.c_float(std))
    return out


def synth_quantize(qtype: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    bb = 144 if qtype == AXF_TYPE_Q4_K else 210
    out = np.empty(x.size // 256 * bb, np.uint8)
    call("axf_synth_quantize", qtype, out.ctypes.data_as(C.c_void_p), x.ctypes.data_as(C.c_void_p),
         C.c_int64(x.size))
    return out


def sampling(temperature: float = 1.0, top_k: int = 40, top_p: float = 1.0,
             rep_penalty: float = 1.0, rep_penalty_last_n: int = 64, seed: int = 42,
             eos_id: int = -1) -> _ffi.Sampling:
    """axf_sampling with LlamaConfig's defaults (models/llama.hpp:18-33) and the
    reference's fixed seed 42."""
    return _ffi.Sampling(float(temperature), int(top_k), float(top_p), float(rep_penalty),
                         int(rep_penalty_last_n), int(seed), int(eos_id))


def mt19937(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    call("axf_mt19937", int(seed), out.ctypes.data_as(C.c_void_p), int(n))
    return out


def sampling_uniforms(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    call("axf_sampling_uniforms", int(seed), out.ctypes.data_as(C.c_void_p), int(n))
    return out


def synth_weight(qtype: int, rows: int, cols: int, seed: int, std: float = 0.02) -> np.ndarray:
    out = np.empty(rows * row_bytes(qtype, cols), np.uint8)
    call("axf_synth_weight", qtype, out.ctypes.data_as(C.c_void_p), C.c_int64(rows), C.c_int64(cols),
         C.c_uint64(seed), C.c_float(std))
    return out


__all__ = [
    "AXF_TYPE_Q4_K",
    "AXF_TYPE_Q6_K",
    "Buffer",
    "Context",
    "Q8_0_BYTES",
    "device_count",
    "rope_table",
    "row_bytes",
    "synth_normal",
    "synth_quantize",
    "synth_weight",
    "_ffi",
]
