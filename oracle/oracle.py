"""ctypes wrapper of the CPU parity oracle — TEST INFRASTRUCTURE ONLY.

Used by tests/, __graft_entry__.smoke() (as the checker) and bench.py's
cpu_baseline leg.  Never used by llm_core_amd.

  orc : liboracle.so, the plain-C restatement (oracle/axf_oracle.c)
  ref : oracle/_ref/libaxf_ref.so, the reference's own x86 kernels compiled
        from their sources (None when it was not built)
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# AXF_ORACLE_LIB: another build of axf_oracle.c (the mutation test's planted
# slips, tests/test_oracle_mutations.py); by default the one built here
ORC_PATH = Path(os.environ["AXF_ORACLE_LIB"]) if os.environ.get("AXF_ORACLE_LIB") else HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libaxf_ref.so"

Q4K, Q6K, F32 = 12, 14, 0
BLOCK_BYTES = {Q4K: 144, Q6K: 210}
Q8_0_BYTES = 36

vp, i32, i64, sz, f32 = C.c_void_p, C.c_int, C.c_int64, C.c_size_t, C.c_float


def _ptr(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


def _load_orc() -> C.CDLL:
    if not ORC_PATH.exists():
        raise ImportError(f"{ORC_PATH} missing: run `make -C oracle`")
    lib = C.CDLL(str(ORC_PATH))
    sig = {
        "orc_fp16_to_fp32": ([C.c_uint16], f32),
        "orc_dequant_q4k": ([vp, vp, i64], None),
        "orc_dequant_q6k": ([vp, vp, i64], None),
        "orc_gemv_q4k_f32": ([vp, vp, vp, i32, i32, i32, sz], None),
        "orc_gemv_q6k_f32": ([vp, vp, vp, i32, i32, i32, sz], None),
        "orc_quantize_q8_0": ([vp, vp, i32], None),
        "orc_gemv_q4k_q8": ([vp, vp, vp, i32, i32, i32, sz], None),
        "orc_gemv_q6k_q8": ([vp, vp, vp, i32, i32, i32, sz], None),
        "orc_repack_q4k_r8": ([vp, vp, i32, i32], None),
        "orc_gemm_q4k_q8": ([vp, vp, vp, i32, i32, i32, sz, i32, i32], None),
        "orc_rmsnorm": ([vp, vp, vp, i32, f32], None),
        "orc_rope_table": ([vp, vp, i32, f32, i32], None),
        "orc_rope": ([vp, vp, i32, i32, i32, vp, vp], None),
        "orc_dot_f32": ([vp, vp, i32], f32),
        "orc_softmax": ([vp, i32], None),
        "orc_attention": ([vp, vp, vp, vp, i32, i32, i32, i32, vp], None),
        "orc_exp_cephes": ([f32], f32),
        "orc_swiglu": ([vp, vp, i32], None),
        "orc_argmax": ([vp, i32], i32),
        "orc_top2_margin": ([vp, i32], f32),
        "orc_rep_penalty": ([vp, i32, vp, i32, i32, f32], None),
        "orc_gemv_q8_0w_q8": ([vp, vp, vp, i32, i32, i32, sz], None),
        "orc_gemv_q8_0w_f32": ([vp, vp, vp, i32, i32, i32, sz], None),
        "orc_gemv_q5_0_f32": ([vp, vp, vp, i32, i32, i32, sz], None),
        "orc_gemv_f16_f32": ([vp, vp, vp, vp, i32, i32, i32], None),
        "orc_dequant_row": ([vp, i32, vp, i32], None),
        "orc_sample": ([vp, i32, i32, f32, f32, f32, C.POINTER(f32)], i32),
        "orc_rmsnorm_heads": ([vp, vp, i32, i32, f32], None),
        "orc_state_new": ([vp], vp),
        "orc_state_free": ([vp], None),
        "orc_state_logits": ([vp], C.POINTER(C.c_float)),
        "orc_state_x": ([vp], C.POINTER(C.c_float)),
        "orc_state_kv_k": ([vp], C.POINTER(C.c_float)),
        "orc_state_kv_v": ([vp], C.POINTER(C.c_float)),
        "orc_state_q": ([vp], C.POINTER(C.c_float)),
        "orc_state_attn_out": ([vp], C.POINTER(C.c_float)),
        "orc_state_h": ([vp], C.POINTER(C.c_float)),
        "orc_forward_token": ([vp, vp, i32, i32], None),
        "orc_forward_layer": ([vp, vp, i32, i32], None),
        "orc_forward_batch": ([vp, vp, vp, i32, i32], None),
        "orc_generate_greedy": ([vp, vp, i32, i32, i32, vp, vp], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


def _load_ref() -> C.CDLL | None:
    if not REF_PATH.exists():
        return None
    lib = C.CDLL(str(REF_PATH))
    sig = {
        "ref_has_avxvnni": ([], i32),
        "ref_has_avx2": ([], i32),
        "ref_gemv_q4k_f32": ([vp, vp, vp, i32, i32, i32, sz], None),
        "ref_gemv_q6k_f32": ([vp, vp, vp, i32, i32, i32, sz], None),
        "ref_gemv_f16_f32": ([vp, vp, vp, vp, i32, i32, i32], None),
        "ref_quantize_q8_0": ([vp, vp, i32], None),
        "ref_gemv_q4k_q8": ([vp, vp, vp, i32, i32, i32, sz, i32], None),
        "ref_repack_q4k_r8": ([vp, vp, i32, i32], None),
        "ref_gemv_q4k_r8": ([vp, vp, vp, i32, i32, i32, i32], None),
        "ref_gemv_q6k_q8": ([vp, vp, vp, i32, i32, i32, sz], None),
        "ref_gemm_q4k_q8": ([vp, vp, vp, i32, i32, i32, sz, i32, i32, i32], None),
        "ref_time_decode_gemv": ([i32, C.POINTER(vp), i32, i32, i32, vp, vp, i32, i32,
                                  C.POINTER(i32)], C.c_double),
        "ref_time_decode_step": ([vp, vp, vp, i32, i32, i32, i32, C.POINTER(i32),
                                  C.POINTER(i32)], C.c_double),
        "ref_time_gemv_f32": ([i32, C.POINTER(vp), i32, i32, i32, vp, vp, i32, i32,
                               C.POINTER(i32)], C.c_double),
        "ref_time_gemm_q4k": ([C.POINTER(vp), i32, i32, i32, vp, i32, vp, i32, i32,
                               C.POINTER(i32)], C.c_double),
        "ref_time_head_argmax": ([C.POINTER(vp), i32, i32, i32, vp, vp, i32, i32, C.POINTER(i32),
                                  C.POINTER(i32)], C.c_double),
        "ref_generate_greedy": ([vp, vp, i32, i32, i32, vp, vp, i32, vp, vp], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


orc = _load_orc()
ref = _load_ref()


def row_bytes(qtype: int, cols: int) -> int:
    return (cols // 256) * BLOCK_BYTES[qtype]


# ---- oracle (restatement) -------------------------------------------------

def dequant(qtype: int, blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, np.uint8)
    nb = blocks.size // BLOCK_BYTES[qtype]
    out = np.empty(nb * 256, np.float32)
    fn = orc.orc_dequant_q4k if qtype == Q4K else orc.orc_dequant_q6k
    fn(_ptr(out), _ptr(blocks), nb)
    return out


def gemv_f32(qtype: int, W: np.ndarray, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    fn = orc.orc_gemv_q4k_f32 if qtype == Q4K else orc.orc_gemv_q6k_f32
    fn(_ptr(y), _ptr(W), _ptr(x), 0, rows, cols, row_bytes(qtype, cols))
    return y


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size // 32 * Q8_0_BYTES, np.uint8)
    orc.orc_quantize_q8_0(_ptr(out), _ptr(x), x.size)
    return out


def gemv_q8(qtype: int, W: np.ndarray, xq8: np.ndarray, rows: int, cols: int) -> np.ndarray:
    y = np.empty(rows, np.float32)
    fn = orc.orc_gemv_q4k_q8 if qtype == Q4K else orc.orc_gemv_q6k_q8
    fn(_ptr(y), _ptr(W), _ptr(xq8), 0, rows, cols, row_bytes(qtype, cols))
    return y


def gemm_q4k_q8(W: np.ndarray, XQ8: np.ndarray, rows: int, T: int, cols: int) -> np.ndarray:
    Y = np.empty(T * rows, np.float32)
    orc.orc_gemm_q4k_q8(_ptr(Y), _ptr(W), _ptr(XQ8), rows, T, cols, row_bytes(Q4K, cols), 0, rows)
    return Y.reshape(T, rows)


def repack_r8(W: np.ndarray, rows: int, cols: int) -> np.ndarray:
    out = np.empty(W.size, np.uint8)
    orc.orc_repack_q4k_r8(_ptr(out), _ptr(W), rows, cols)
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    orc.orc_rmsnorm(_ptr(y), _ptr(x), _ptr(w), x.size, eps)
    return y


def rmsnorm_heads(x: np.ndarray, w: np.ndarray, n_heads: int, hd: int, eps: float) -> np.ndarray:
    """rms_norm_heads_inplace (llama_model.cpp:421-429) on a copy."""
    y = np.ascontiguousarray(x, np.float32).copy()
    w = np.ascontiguousarray(w, np.float32)
    orc.orc_rmsnorm_heads(_ptr(y), _ptr(w), n_heads, hd, eps)
    return y


def rope_table(hd: int, theta: float, max_pos: int) -> tuple[np.ndarray, np.ndarray]:
    c = np.empty(max_pos * (hd // 2), np.float32)
    s = np.empty_like(c)
    orc.orc_rope_table(_ptr(c), _ptr(s), hd, theta, max_pos)
    return c, s


def rope(x: np.ndarray, pos: int, n_heads: int, hd: int, cos_t: np.ndarray,
         sin_t: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    orc.orc_rope(_ptr(y), _ptr(x), pos, n_heads, hd, _ptr(cos_t), _ptr(sin_t))
    return y


def attention(q, kc, vc, seq, n_heads, n_kv_heads, hd) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    kc = np.ascontiguousarray(kc, np.float32)
    vc = np.ascontiguousarray(vc, np.float32)
    out = np.empty(n_heads * hd, np.float32)
    scores = np.empty(max(seq, 1), np.float32)
    orc.orc_attention(_ptr(out), _ptr(q), _ptr(kc), _ptr(vc), seq, n_heads, n_kv_heads, hd,
                      _ptr(scores))
    return out


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.array(g, np.float32, copy=True)
    u = np.ascontiguousarray(u, np.float32)
    orc.orc_swiglu(_ptr(g), _ptr(u), g.size)
    return g


def argmax(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, np.float32)
    return int(orc.orc_argmax(_ptr(x), x.size))


def ref_time_decode_gemv(qtype: int, W: np.ndarray, rows: int, cols: int, x: np.ndarray,
                         n_copies: int, iters: int, n_threads: int = 0):
    """Median seconds per reference decode GEMV (quantize + r8/4-row kernel on the
    reference ThreadPool), weights rotated over n_copies host buffers."""
    assert ref is not None, "oracle/_ref not built"
    if qtype == Q4K:
        W = repack_r8(W, rows, cols)  # the reference repacks at load (llama_model.cpp:963-971)
    copies = [W] + [W.copy() for _ in range(n_copies - 1)]
    arr = (C.c_void_p * n_copies)(*[c.ctypes.data for c in copies])
    y = np.empty(rows, np.float32)
    used = C.c_int(0)
    x = np.ascontiguousarray(x, np.float32)
    t = ref.ref_time_decode_gemv(qtype, arr, n_copies, rows, cols, _ptr(x), _ptr(y), iters,
                                 n_threads, C.byref(used))
    return t, used.value


def _copies(W: np.ndarray, min_bytes: int):
    n = max(2, -(-min_bytes // max(W.nbytes, 1)))
    copies = [W] + [W.copy() for _ in range(n - 1)]
    return copies, (C.c_void_p * n)(*[c.ctypes.data for c in copies]), n


def ref_time_gemv_f32(qtype: int, W: np.ndarray, rows: int, cols: int, x: np.ndarray,
                      iters: int, min_bytes: int = 640 << 20, n_threads: int = 0):
    """Median seconds of the reference's fp32-activation GEMV (gemv_wt) over
    weight copies rotated past min_bytes; (seconds, threads)."""
    assert ref is not None, "oracle/_ref not built"
    keep, arr, n = _copies(np.ascontiguousarray(W), min_bytes)
    y = np.empty(rows, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    used = C.c_int(0)
    t = ref.ref_time_gemv_f32(qtype, arr, n, rows, cols, _ptr(x), _ptr(y), iters, n_threads,
                              C.byref(used))
    del keep
    return t, used.value


def ref_time_gemm_q4k(W: np.ndarray, rows: int, cols: int, XQ8: np.ndarray, T: int, iters: int,
                      min_bytes: int = 640 << 20, n_threads: int = 0):
    """Median seconds of the reference's T-token Q4_K GEMM (gemm_wt_q8)."""
    assert ref is not None, "oracle/_ref not built"
    keep, arr, n = _copies(np.ascontiguousarray(W), min_bytes)
    Y = np.empty(T * rows, np.float32)
    XQ8 = np.ascontiguousarray(XQ8)
    used = C.c_int(0)
    t = ref.ref_time_gemm_q4k(arr, n, rows, cols, _ptr(XQ8), T, _ptr(Y), iters, n_threads,
                              C.byref(used))
    del keep
    return t, used.value


def ref_time_head_argmax(W: np.ndarray, rows: int, cols: int, x: np.ndarray, iters: int,
                         min_bytes: int = 640 << 20, n_threads: int = 0):
    """Median seconds of Q8_0 quantise + Q6_K head GEMV + greedy pick; (s, threads, argmax)."""
    assert ref is not None, "oracle/_ref not built"
    keep, arr, n = _copies(np.ascontiguousarray(W), min_bytes)
    y = np.empty(rows, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    used, am = C.c_int(0), C.c_int(0)
    t = ref.ref_time_head_argmax(arr, n, rows, cols, _ptr(x), _ptr(y), iters, n_threads,
                                 C.byref(used), C.byref(am))
    del keep
    return t, used.value, am.value


def ref_time_decode_step(model: "OracleModel", kv_k: np.ndarray, kv_v: np.ndarray, pos: int,
                         warmup: int, steps: int, n_threads: int = 0):
    """Median seconds per reference decode step (see ref_shim.cpp)."""
    assert ref is not None, "oracle/_ref not built"
    used, last = C.c_int(0), C.c_int(0)
    t = ref.ref_time_decode_step(C.byref(model.m), _ptr(kv_k), _ptr(kv_v), pos, warmup, steps,
                                 n_threads, C.byref(used), C.byref(last))
    return t, used.value, last.value


def ref_generate_greedy(model: "OracleModel", prompt, n_gen: int, n_threads: int = 0, top_k: int = 0):
    """Greedy generation of llama_generate_cpu_impl (batched prefill of the
    prompt as given, then one decode step per token) on the reference's
    compiled kernels and ThreadPool (ref_shim.cpp): (ids, top-1 minus top-2
    margins of the logits each id was taken from), and with top_k > 0 also
    each step's top_k (ids, logits), largest first.  Q4_K / Q6_K layer
    matrices."""
    assert ref is not None, "oracle/_ref not built"
    p = np.ascontiguousarray(prompt, np.int32)
    toks = np.zeros(max(n_gen, 1), np.int32)
    margins = np.zeros(max(n_gen, 1), np.float32)
    tk = max(top_k, 1)
    tids = np.zeros((max(n_gen, 1), tk), np.int32)
    tvals = np.zeros((max(n_gen, 1), tk), np.float32)
    n = ref.ref_generate_greedy(C.byref(model.m), _ptr(p), p.size, n_gen, n_threads, _ptr(toks),
                                _ptr(margins), top_k, _ptr(tids), _ptr(tvals))
    if top_k > 0:
        return toks[:n], margins[:n], tids[:n], tvals[:n]
    return toks[:n], margins[:n]


MISC_BLOCK = {8: 34, 6: 22}  # bytes per 32 elements: Q8_0, Q5_0


def misc_row_bytes(qtype: int, cols: int) -> int:
    return cols * 2 if qtype == 1 else (cols + 31) // 32 * MISC_BLOCK[qtype]


def gemv_misc(qtype: int, W: np.ndarray, x: np.ndarray, rows: int, cols: int,
              bias: np.ndarray | None = None) -> np.ndarray:
    """Other weight types with fp32 activations: Q8_0 (q8_0_weight_dot_row),
    Q5_0 (q5_0_dot_row), F16 (gemv_f16_avx2_range)."""
    y = np.zeros(rows, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    W = np.ascontiguousarray(W)
    if qtype == 1:
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        orc.orc_gemv_f16_f32(_ptr(y), _ptr(W), _ptr(x), None if b is None else _ptr(b), 0, rows, cols)
    elif qtype == 8:
        orc.orc_gemv_q8_0w_f32(_ptr(y), _ptr(W), _ptr(x), 0, rows, cols, misc_row_bytes(8, cols))
    else:
        orc.orc_gemv_q5_0_f32(_ptr(y), _ptr(W), _ptr(x), 0, rows, cols, misc_row_bytes(6, cols))
    return y


def gemv_q8_0w_q8(W: np.ndarray, xq8: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """q8_0_weight_dot_q8_row over rows (llama_model.cpp:171-228)."""
    y = np.zeros(rows, np.float32)
    W = np.ascontiguousarray(W)
    xq8 = np.ascontiguousarray(xq8)
    orc.orc_gemv_q8_0w_q8(_ptr(y), _ptr(W), _ptr(xq8), 0, rows, cols, misc_row_bytes(8, cols))
    return y


def dequant_row(qtype: int, row: np.ndarray, cols: int) -> np.ndarray:
    out = np.zeros(cols, np.float32)
    r = np.ascontiguousarray(row)
    orc.orc_dequant_row(_ptr(out), qtype, _ptr(r), cols)
    return out


def rep_penalty(logits: np.ndarray, hist, last_n: int, penalty: float) -> np.ndarray:
    """apply_rep_penalty (llama_model.cpp:1595-1605) on a copy."""
    y = np.ascontiguousarray(logits, np.float32).copy()
    h = np.ascontiguousarray(hist, np.int32)
    orc.orc_rep_penalty(_ptr(y), y.size, _ptr(h), h.size, int(last_n), float(penalty))
    return y


def sample(logits: np.ndarray, top_k: int, top_p: float, temperature: float,
           r: float) -> tuple[int, float]:
    """sample() (llama_model.cpp:1466-1498) with the uniform draw r: (token,
    distance of the decision from flipping)."""
    x = np.ascontiguousarray(logits, np.float32)
    m = C.c_float()
    tok = orc.orc_sample(_ptr(x), x.size, int(top_k), float(top_p), float(temperature),
                         float(r), C.byref(m))
    return int(tok), float(m.value)


def top2_margin(x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, np.float32)
    return float(orc.orc_top2_margin(_ptr(x), x.size))


# ---- oracle decoder ---------------------------------------------------------

class OrcWt(C.Structure):
    _fields_ = [("type", C.c_int), ("data", C.c_void_p)]


class OrcLayer(C.Structure):
    _fields_ = [("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p)] + [
        (n, OrcWt) for n in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown")
    ] + [("bq", C.c_void_p), ("bk", C.c_void_p), ("bv", C.c_void_p), ("q_norm", C.c_void_p),
         ("k_norm", C.c_void_p)]


class OrcModel(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layer", "n_embd", "n_heads", "n_kv_heads", "ffn_dim",
                                        "n_vocab", "n_ctx")] + [
        ("rms_eps", C.c_float), ("rope_theta", C.c_float), ("tok_embd", OrcWt),
        ("output_norm", C.c_void_p), ("output", OrcWt), ("layers", C.POINTER(OrcLayer)),
        ("qk_norm_order", C.c_int)]


class OracleModel:
    """The oracle's decoder over the same host tensors a SynthLlama holds."""

    def __init__(self, hp, tensors: dict):
        self.hp = hp
        self._keep = []

        def arr(name):
            qt, a = tensors[name]
            a = np.ascontiguousarray(a)
            self._keep.append(a)
            return qt, a.ctypes.data

        def wt(name):
            qt, p = arr(name)
            return OrcWt(qt, p)

        def opt(name):
            return arr(name)[1] if name in tensors else None

        layers = (OrcLayer * hp.n_layer)()
        for i in range(hp.n_layer):
            b = f"blk.{i}."
            L = layers[i]
            L.attn_norm = arr(b + "attn_norm.weight")[1]
            L.ffn_norm = arr(b + "ffn_norm.weight")[1]
            for field_name, t in (("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"),
                                  ("wo", "attn_output"), ("wgate", "ffn_gate"),
                                  ("wup", "ffn_up"), ("wdown", "ffn_down")):
                setattr(L, field_name, wt(b + t + ".weight"))
            L.bq = opt(b + "attn_q.bias")
            L.bk = opt(b + "attn_k.bias")
            L.bv = opt(b + "attn_v.bias")
            L.q_norm = opt(b + "attn_q_norm.weight")
            L.k_norm = opt(b + "attn_k_norm.weight")
        self._layers = layers
        out_name = "output.weight" if "output.weight" in tensors else "token_embd.weight"
        self.m = OrcModel(hp.n_layer, hp.n_embd, hp.n_heads, hp.n_kv_heads, hp.ffn_dim,
                          hp.n_vocab, hp.n_ctx, hp.rms_eps, hp.rope_theta,
                          wt("token_embd.weight"), arr("output_norm.weight")[1], wt(out_name),
                          layers, int(getattr(hp, "qk_norm_order", 0)))
        self.state = orc.orc_state_new(C.byref(self.m))

    def close(self):
        if self.state:
            orc.orc_state_free(self.state)
            self.state = None

    def reset(self):
        self.close()
        self.state = orc.orc_state_new(C.byref(self.m))

    def kv_view(self):
        hp = self.hp
        n = hp.n_layer * hp.n_ctx * hp.n_kv_heads * hp.head_dim
        shape = (hp.n_layer, hp.n_ctx, hp.n_kv_heads * hp.head_dim)
        k = np.ctypeslib.as_array(orc.orc_state_kv_k(self.state), (n,)).reshape(shape)
        v = np.ctypeslib.as_array(orc.orc_state_kv_v(self.state), (n,)).reshape(shape)
        return k, v

    def x_view(self):
        return np.ctypeslib.as_array(orc.orc_state_x(self.state), (self.hp.n_embd,))

    def q_view(self):
        """q of the last forward_layer, after bias and RoPE."""
        hp = self.hp
        return np.ctypeslib.as_array(orc.orc_state_q(self.state), (hp.n_heads * hp.head_dim,))

    def attn_out_view(self):
        hp = self.hp
        return np.ctypeslib.as_array(orc.orc_state_attn_out(self.state),
                                     (hp.n_heads * hp.head_dim,))

    def h_view(self):
        """SwiGLU output of the last forward_layer (the down projection's input)."""
        return np.ctypeslib.as_array(orc.orc_state_h(self.state), (self.hp.ffn_dim,))

    def logits(self):
        return np.ctypeslib.as_array(orc.orc_state_logits(self.state), (self.hp.n_vocab,)).copy()

    def forward_layer(self, layer, pos):
        orc.orc_forward_layer(C.byref(self.m), self.state, layer, pos)

    def forward_token(self, token, pos):
        orc.orc_forward_token(C.byref(self.m), self.state, token, pos)

    def forward_batch(self, tokens, pos_start=0):
        t = np.ascontiguousarray(tokens, np.int32)
        orc.orc_forward_batch(C.byref(self.m), self.state, _ptr(t), t.size, pos_start)

    def generate(self, prompt, n_gen, batched_prefill=True):
        p = np.ascontiguousarray(prompt, np.int32)
        toks = np.zeros(max(n_gen, 1), np.int32)
        margins = np.zeros(max(n_gen, 1), np.float32)
        n = orc.orc_generate_greedy(C.byref(self.m), _ptr(p), p.size, n_gen,
                                    1 if batched_prefill else 0, _ptr(toks), _ptr(margins))
        return toks[:n], margins[:n]
