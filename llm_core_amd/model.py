"""Synthetic LLaMA-family models and the device decoder handle.

SynthLlama draws every weight N(0, std) from a seed and quantizes it with the
Q4_K_M mix of the reference's benchmarks (Q4_K: token_embd, attn_q, attn_k,
attn_output, ffn_gate, ffn_up; Q6_K: attn_v, ffn_down, output); norm weights
are 1.0 unless norm_std > 0 (also the per-head q/k norm weights of a model
with qk_norm_order != 0).  LlamaHip uploads such a model once and drives the
decode step on the GPU through the C-ABI.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _ffi, hip
from ._ffi import (AXF_TYPE_F16, AXF_TYPE_F32, AXF_TYPE_Q4_K, AXF_TYPE_Q5_0, AXF_TYPE_Q6_K,
                   AXF_TYPE_Q8_0, LlamaHparams, call, lib)


@dataclass
class Hparams:
    n_layer: int
    n_embd: int
    n_heads: int
    n_kv_heads: int
    ffn_dim: int
    n_vocab: int
    n_ctx: int
    rms_eps: float = 1e-5
    rope_theta: float = 10000.0
    qk_norm_order: int = 0  # per-head q/k RMSNorm: 0 none, 1 before RoPE (qwen3), 2 after

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_heads

    def to_c(self) -> LlamaHparams:
        return LlamaHparams(self.n_layer, self.n_embd, self.n_heads, self.n_kv_heads,
                            self.ffn_dim, self.n_vocab, self.n_ctx, self.rms_eps, self.rope_theta,
                            self.qk_norm_order)


# LLaMA-2-7B architecture (the decode benchmark) and a Qwen2.5-3B-like layer
# (hidden 2048, 16/2 heads, FFN 11008: tests/test_gguf_reader.cpp:429-444 of the reference)
LLAMA2_7B = dict(n_layer=32, n_embd=4096, n_heads=32, n_kv_heads=32, ffn_dim=11008,
                 n_vocab=32000, rms_eps=1e-5, rope_theta=10000.0)
QWEN25_3B_LAYER = dict(n_layer=1, n_embd=2048, n_heads=16, n_kv_heads=2, ffn_dim=11008,
                       n_vocab=151936, rms_eps=1e-6, rope_theta=1e6)

# Qwen2.5-0.5B shape (qwen2 architecture: q/k/v biases, tied embeddings)
QWEN25_05B = dict(n_layer=24, n_embd=896, n_heads=14, n_kv_heads=2, ffn_dim=4864,
                  n_vocab=151936, rms_eps=1e-6, rope_theta=1e6)

Q4K_M_TYPES = {
    "attn_q": AXF_TYPE_Q4_K,
    "attn_k": AXF_TYPE_Q4_K,
    "attn_v": AXF_TYPE_Q6_K,
    "attn_output": AXF_TYPE_Q4_K,
    "ffn_gate": AXF_TYPE_Q4_K,
    "ffn_up": AXF_TYPE_Q4_K,
    "ffn_down": AXF_TYPE_Q6_K,
}


def q4k_m_fallback_types(layer: int, n_layer: int) -> dict:
    """The weight types llama.cpp's Q4_K_M mix gives a model whose hidden size
    is not a multiple of 256 (Qwen2.5-0.5B: 896): matrices with 896-wide rows
    fall back from Q4_K to Q5_0 and from Q6_K to Q8_0; ffn_down (4864-wide rows)
    keeps Q6_K on the layers that get more bits (the first and last eighth and
    every third layer between), Q4_K elsewhere."""
    more = layer < n_layer // 8 or layer >= 7 * n_layer // 8 or (layer - n_layer // 8) % 3 == 2
    return {"attn_q": AXF_TYPE_Q5_0, "attn_k": AXF_TYPE_Q5_0,
            "attn_v": AXF_TYPE_Q8_0 if more else AXF_TYPE_Q5_0,
            "attn_output": AXF_TYPE_Q5_0, "ffn_gate": AXF_TYPE_Q5_0, "ffn_up": AXF_TYPE_Q5_0,
            "ffn_down": AXF_TYPE_Q6_K if more else AXF_TYPE_Q4_K}


def synth_other(qtype: int, rows: int, cols: int, seed: int, std: float = 0.02) -> np.ndarray:
    """N(0, std) rows in the other GGUF weight types (F16, Q8_0, Q5_0), quantised
    with ggml's reference rounding: Q8_0 d = amax/127, q = round(x/d); Q5_0
    d = m/-16 for the value m of largest magnitude, q = min(31, int(x/d + 16.5))."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, cols)) * std).astype(np.float32)
    if qtype == AXF_TYPE_F16:
        return x.astype(np.float16).reshape(-1).view(np.uint8)
    b = x.reshape(rows, cols // 32, 32)
    if qtype == AXF_TYPE_Q8_0:
        d = (np.abs(b).max(axis=2) / 127.0).astype(np.float16)
        df = d.astype(np.float32)[..., None]
        q = np.clip(np.round(np.divide(b, df, out=np.zeros_like(b), where=df != 0)), -127, 127)
        return np.concatenate([d.view(np.uint8).reshape(rows, -1, 2),
                               q.astype(np.int8).view(np.uint8)], axis=2).reshape(-1)
    idx = np.abs(b).argmax(axis=2)[..., None]
    m = np.take_along_axis(b, idx, axis=2)[..., 0]
    d = (m / -16.0).astype(np.float16)
    inv = np.divide(1.0, d.astype(np.float32), out=np.zeros(d.shape, np.float32),
                    where=d.astype(np.float32) != 0)[..., None]
    q = np.minimum(31, (b * inv + 16.5).astype(np.int32)).astype(np.uint32)
    lo, hi = q[..., :16], q[..., 16:]
    qs = ((lo & 15) | ((hi & 15) << 4)).astype(np.uint8)
    bits = np.arange(16, dtype=np.uint32)
    qh = (((lo >> 4) & 1) << bits).sum(axis=2) + (((hi >> 4) & 1) << (bits + 16)).sum(axis=2)
    return np.concatenate([d.view(np.uint8).reshape(rows, -1, 2),
                           qh.astype(np.uint32).view(np.uint8).reshape(rows, -1, 4), qs],
                          axis=2).reshape(-1)


@dataclass
class SynthLlama:
    hp: Hparams
    seed: int = 5
    std: float = 0.02
    norm_std: float = 0.0
    with_bias: bool = False
    embd_type: int = AXF_TYPE_Q4_K   # token_embd.weight
    head_type: int = AXF_TYPE_Q6_K   # output.weight; None: tied to token_embd (no output.weight)
    layer_types: object = None       # {base: qtype} or layer -> {base: qtype}; default Q4K_M_TYPES
    tensors: dict = field(default_factory=dict)  # name -> (qtype, ndarray)

    def __post_init__(self) -> None:
        hp = self.hp
        E, FD, hd = hp.n_embd, hp.ffn_dim, hp.head_dim
        qo, kvo = hp.n_heads * hd, hp.n_kv_heads * hd
        k = 0

        def seed() -> int:
            nonlocal k
            k += 1
            return self.seed * 1000003 + k

        def qw(name: str, qtype: int, rows: int, cols: int) -> None:
            if qtype in (AXF_TYPE_Q4_K, AXF_TYPE_Q6_K):
                a = hip.synth_weight(qtype, rows, cols, seed(), self.std)
            else:
                a = synth_other(qtype, rows, cols, seed(), self.std)
            self.tensors[name] = (qtype, a)

        def norm(name: str, n: int) -> None:
            if self.norm_std > 0:
                v = hip.synth_normal(n, seed(), 1.0, self.norm_std)
            else:
                v = np.ones(n, np.float32)
            self.tensors[name] = (AXF_TYPE_F32, v)

        qw("token_embd.weight", self.embd_type, hp.n_vocab, E)
        if self.head_type is not None:
            qw("output.weight", self.head_type, hp.n_vocab, E)
        norm("output_norm.weight", E)
        shapes = {"attn_q": (qo, E), "attn_k": (kvo, E), "attn_v": (kvo, E),
                  "attn_output": (E, qo), "ffn_gate": (FD, E), "ffn_up": (FD, E),
                  "ffn_down": (E, FD)}
        for layer in range(hp.n_layer):
            norm(f"blk.{layer}.attn_norm.weight", E)
            norm(f"blk.{layer}.ffn_norm.weight", E)
            lt = self.layer_types(layer) if callable(self.layer_types) else self.layer_types
            for base, (rows, cols) in shapes.items():
                qw(f"blk.{layer}.{base}.weight", (lt or {}).get(base, Q4K_M_TYPES[base]), rows, cols)
            if self.with_bias:
                for base, n in (("attn_q", qo), ("attn_k", kvo), ("attn_v", kvo)):
                    self.tensors[f"blk.{layer}.{base}.bias"] = (
                        AXF_TYPE_F32, hip.synth_normal(n, seed(), 0.0, 0.02))
            if hp.qk_norm_order:
                norm(f"blk.{layer}.attn_q_norm.weight", hd)
                norm(f"blk.{layer}.attn_k_norm.weight", hd)

    def weight_bytes_per_token(self) -> int:
        """Bytes of quantized and norm weights one decode step reads (one embedding row)."""
        total = 0
        for name, (qt, arr) in self.tensors.items():
            if name == "token_embd.weight":
                total += hip.row_bytes(qt, self.hp.n_embd)
                if "output.weight" not in self.tensors:  # tied head: the whole matrix
                    total += arr.nbytes
            else:
                total += arr.nbytes
        return total


class LlamaHip:
    """Device-resident decoder (axf_llama_* in include/axf_hip.h)."""

    def __init__(self, ctx: hip.Context, model: SynthLlama):
        self.ctx = ctx
        self.hp = model.hp
        h = C.c_void_p()
        hpc = model.hp.to_c()
        call("axf_llama_create", ctx.handle, C.byref(hpc), C.byref(h))
        self.handle = h
        keep = []
        for name, (qt, arr) in model.tensors.items():
            a = np.ascontiguousarray(arr)
            keep.append(a)
            call("axf_llama_set_tensor", self.handle, name.encode(), qt,
                 a.ctypes.data_as(C.c_void_p), C.c_size_t(a.nbytes))
        call("axf_llama_load", self.handle)
        del keep

    @classmethod
    def from_gguf(cls, ctx: hip.Context, path, max_context_len: int = 0) -> "LlamaHip":
        """Load a GGUF file onto the device (axf_llama_from_gguf): hyperparameters
        from its metadata, weights uploaded from the file mapping."""
        self = cls.__new__(cls)
        self.ctx = ctx
        h = C.c_void_p()
        call("axf_llama_from_gguf", ctx.handle, str(path).encode(), int(max_context_len),
             C.byref(h))
        self.handle = h
        c = LlamaHparams()
        call("axf_llama_get_hparams", self.handle, C.byref(c))
        self.hp = Hparams(c.n_layer, c.n_embd, c.n_heads, c.n_kv_heads, c.ffn_dim, c.n_vocab,
                          c.n_ctx, c.rms_eps, c.rope_theta, c.qk_norm_order)
        return self

    def close(self) -> None:
        if self.handle:
            call("axf_llama_destroy", self.handle)
            self.handle = None

    def __enter__(self) -> "LlamaHip":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def device_bytes(self) -> int:
        return int(lib.axf_llama_device_bytes(self.handle))

    def set_x(self, x: np.ndarray) -> None:
        a = np.ascontiguousarray(x, np.float32)
        call("axf_llama_set_x", self.handle, a.ctypes.data_as(C.c_void_p))

    def get_x(self) -> np.ndarray:
        out = np.empty(self.hp.n_embd, np.float32)
        call("axf_llama_get_x", self.handle, out.ctypes.data_as(C.c_void_p))
        return out

    def set_kv(self, layer: int, k: np.ndarray, v: np.ndarray, n_pos: int) -> None:
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        call("axf_llama_set_kv", self.handle, layer, k.ctypes.data_as(C.c_void_p),
             v.ctypes.data_as(C.c_void_p), n_pos)

    def fill_kv_random(self, n_pos: int, seed: int) -> None:
        call("axf_llama_fill_kv_random", self.handle, n_pos, C.c_uint64(seed))

    def logits(self) -> np.ndarray:
        out = np.empty(self.hp.n_vocab, np.float32)
        call("axf_llama_get_logits", self.handle, out.ctypes.data_as(C.c_void_p))
        return out

    def forward_layer(self, layer: int, pos: int) -> None:
        call("axf_llama_forward_layer", self.handle, layer, pos)

    def forward_layer_stages(self, layer: int, pos: int, first: int, last: int) -> None:
        """Stages first..last (1 q|k|v, 2 attention, 3 o, 4 gate|up+SwiGLU,
        5 down) of one layer, with the decode step's fused kernels."""
        call("axf_llama_forward_layer_stages", self.handle, layer, pos, first, last)

    def buffer(self, which: int) -> np.ndarray:
        """A decoder buffer (AXF_LLAMA_BUF_*): fp32, or uint8 for ATTN_Q8."""
        hp = self.hp
        qo, kvo = hp.n_heads * hp.head_dim, hp.n_kv_heads * hp.head_dim
        shape = {_ffi.AXF_LLAMA_BUF_X: (np.float32, hp.n_embd),
                 _ffi.AXF_LLAMA_BUF_QKV: (np.float32, qo + 2 * kvo),
                 _ffi.AXF_LLAMA_BUF_ATTN: (np.float32, qo),
                 _ffi.AXF_LLAMA_BUF_ATTN_Q8: (np.uint8, qo // 32 * 36),
                 _ffi.AXF_LLAMA_BUF_H: (np.float32, hp.ffn_dim),
                 _ffi.AXF_LLAMA_BUF_LOGITS: (np.float32, hp.n_vocab)}[which]
        out = np.empty(shape[1], shape[0])
        call("axf_llama_get_buffer", self.handle, which, out.ctypes.data_as(C.c_void_p),
             C.c_size_t(out.nbytes))
        return out

    def get_kv(self, layer: int, pos0: int, n_pos: int) -> tuple[np.ndarray, np.ndarray]:
        kve = self.hp.n_kv_heads * self.hp.head_dim
        k = np.empty((n_pos, kve), np.float32)
        v = np.empty((n_pos, kve), np.float32)
        call("axf_llama_get_kv", self.handle, layer, k.ctypes.data_as(C.c_void_p),
             v.ctypes.data_as(C.c_void_p), pos0, n_pos)
        return k, v

    def forward_token(self, token: int, pos: int) -> None:
        call("axf_llama_forward_token", self.handle, token, pos)

    def forward_batch(self, tokens, pos_start: int = 0) -> None:
        """Batched prefill of `tokens` at positions pos_start.. (llama_forward_batch)."""
        t = np.ascontiguousarray(tokens, np.int32)
        call("axf_llama_forward_batch", self.handle, t.ctypes.data_as(C.c_void_p), int(t.size),
             pos_start)

    def generate_sampled(self, prompt, max_new_tokens: int, use_graph: bool = True,
                         **sampling) -> np.ndarray:
        """llama_generate_cpu_impl's loop with the device sampler
        (axf_llama_generate_sampled); keyword arguments as hip.sampling()."""
        p = np.ascontiguousarray(prompt, np.int32)
        s = hip.sampling(**sampling)
        out = np.zeros(max(1, max_new_tokens), np.int32)
        n = C.c_int()
        call("axf_llama_generate_sampled", self.handle, p.ctypes.data_as(C.c_void_p), p.size,
             int(max_new_tokens), C.byref(s), out.ctypes.data_as(C.c_void_p), C.byref(n),
             1 if use_graph else 0)
        return out[:n.value].copy()

    def generate(self, prompt, n_gen: int, use_graph: bool = True,
                 batched_prefill: bool = True) -> np.ndarray:
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(n_gen, 1), np.int32)
        call("axf_llama_generate_ex", self.handle, p.ctypes.data_as(C.c_void_p), int(p.size),
             n_gen, out.ctypes.data_as(C.c_void_p), 1 if use_graph else 0,
             1 if batched_prefill else 0)
        return out[:n_gen]

    def bench_prefill(self, n_tokens: int, reps: int = 3) -> float:
        """Mean milliseconds of a batched prefill of n_tokens synthetic tokens."""
        ms = C.c_float(0)
        call("axf_llama_bench_prefill", self.handle, n_tokens, reps, C.byref(ms))
        return ms.value

    def bench_decode(self, pos: int, warmup: int, steps: int) -> float:
        """Milliseconds for `steps` graph-replayed decode steps at position `pos`."""
        ms = C.c_float(0)
        call("axf_llama_bench_decode", self.handle, pos, warmup, steps, C.byref(ms))
        return ms.value

    def bench_stage(self, stage: int, pos: int, reps: int) -> float:
        """Milliseconds for `reps` passes of decode stage `stage` (1 q|k|v, 2
        attention, 3 o, 4 gate|up, 5 down, 6 head) over every layer."""
        ms = C.c_float(0)
        call("axf_llama_bench_stage", self.handle, stage, pos, reps, C.byref(ms))
        return ms.value
