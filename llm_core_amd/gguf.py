"""GGUF v2/v3 files: a writer for synthetic models and the reader of
include/axf_hip.h (axf_gguf_*, the counterpart of the reference's GgufReader,
src/loader/gguf_reader.hpp).

The writer lays a file out as the format defines it (the layout the
reference's parser walks, gguf_loader.cpp:1-20): "GGUF", u32 version, i64
tensor count, i64 KV count, the KV pairs (string key, i32 type tag, value;
arrays as i32 element tag + u64 count + elements), the tensor infos (string
name, u32 n_dims, i64 dims innermost first, i32 GGML type, u64 offset into
the data blob), zero padding to the alignment, then the data blob with every
tensor at an aligned offset.
"""
from __future__ import annotations

import ctypes as C
import struct
from pathlib import Path

import numpy as np

from ._ffi import GgufModelConfig, GgufTensor, call, lib

# GGUF value type tags
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_POD = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<b",
        U64: "<Q", I64: "<q", F64: "<d"}

# GGML tensor types used by the decoder
GGML_F32, GGML_Q4_K, GGML_Q6_K = 0, 12, 14


def _str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


class GGUFWriter:
    """Build a GGUF file in memory.  Values are written with explicit type tags;
    `raw_kv` / `raw_tensor_info` allow malformed entries for parser tests."""

    def __init__(self, version: int = 3, alignment: int = 32, magic: bytes = b"GGUF"):
        self.version = version
        self.alignment = alignment
        self.magic = magic
        self.kv: list[bytes] = []
        self.infos: list[bytes] = []
        self.blobs: list[tuple[int, bytes]] = []  # (offset, bytes)
        self.blob_end = 0

    # ---- KV pairs ----
    def add(self, key: str, tag: int, value) -> "GGUFWriter":
        self.kv.append(_str(key) + struct.pack("<i", tag) + self._value(tag, value))
        return self

    def add_array(self, key: str, elem_tag: int, values) -> "GGUFWriter":
        body = struct.pack("<iQ", elem_tag, len(values))
        body += b"".join(self._value(elem_tag, v) for v in values)
        self.kv.append(_str(key) + struct.pack("<i", ARRAY) + body)
        return self

    def raw_kv(self, payload: bytes) -> "GGUFWriter":
        self.kv.append(payload)
        return self

    @staticmethod
    def _value(tag: int, v) -> bytes:
        if tag == STRING:
            return _str(v)
        if tag == BOOL:
            return struct.pack("<b", 1 if v else 0)
        return struct.pack(_POD[tag], v)

    # ---- tensors ----
    def add_tensor(self, name: str, data, ggml_type: int, shape) -> "GGUFWriter":
        """shape in GGML order (innermost first): a [rows][cols] matrix is (cols, rows)."""
        b = data.tobytes() if isinstance(data, np.ndarray) else bytes(data)
        off = -(-self.blob_end // self.alignment) * self.alignment
        self.infos.append(_str(name) + struct.pack("<I", len(shape)) +
                          b"".join(struct.pack("<q", int(d)) for d in shape) +
                          struct.pack("<iQ", ggml_type, off))
        self.blobs.append((off, b))
        self.blob_end = off + len(b)
        return self

    def raw_tensor_info(self, payload: bytes) -> "GGUFWriter":
        self.infos.append(payload)
        return self

    def to_bytes(self, n_tensors: int | None = None, n_kv: int | None = None) -> bytes:
        head = self.magic + struct.pack("<Iqq", self.version,
                                        len(self.infos) if n_tensors is None else n_tensors,
                                        len(self.kv) if n_kv is None else n_kv)
        meta = head + b"".join(self.kv) + b"".join(self.infos)
        meta += b"\0" * (-len(meta) % self.alignment)
        blob = bytearray(self.blob_end)
        for off, b in self.blobs:
            blob[off:off + len(b)] = b
        return meta + bytes(blob)

    def write(self, path: str | Path, **kw) -> Path:
        p = Path(path)
        p.write_bytes(self.to_bytes(**kw))
        return p


def llama_gguf(model, arch: str = "llama", tokens: bool = True, tied: bool = False,
               context_length: int | None = None, version: int = 3) -> GGUFWriter:
    """A GGUF image of a synthetic model (`model.SynthLlama`): the metadata keys
    Engine::from_gguf reads (src/engine.cpp:85-118) and every tensor, matrices
    as (cols, rows) in GGML order.  tied=True leaves out output.weight (the
    head then reuses token_embd, llama_model.cpp:979)."""
    hp = model.hp
    w = GGUFWriter(version=version)
    w.add("general.architecture", STRING, arch)
    w.add(f"{arch}.block_count", U32, hp.n_layer)
    w.add(f"{arch}.embedding_length", U32, hp.n_embd)
    w.add(f"{arch}.feed_forward_length", U32, hp.ffn_dim)
    w.add(f"{arch}.attention.head_count", U32, hp.n_heads)
    w.add(f"{arch}.attention.head_count_kv", U32, hp.n_kv_heads)
    w.add(f"{arch}.context_length", U32, hp.n_ctx if context_length is None else context_length)
    w.add(f"{arch}.attention.layer_norm_rms_epsilon", F32, hp.rms_eps)
    w.add(f"{arch}.rope.freq_base", F32, hp.rope_theta)
    w.add("tokenizer.ggml.bos_token_id", U32, 1)
    w.add("tokenizer.ggml.eos_token_id", U32, 2)
    if tokens:
        w.add_array("tokenizer.ggml.tokens", STRING, [f"<t{i}>" for i in range(hp.n_vocab)])
    E, FD, hd = hp.n_embd, hp.ffn_dim, hp.n_embd // hp.n_heads
    qo, kvo = hp.n_heads * hd, hp.n_kv_heads * hd
    dims = {"token_embd": (hp.n_vocab, E), "output": (hp.n_vocab, E), "attn_q": (qo, E),
            "attn_k": (kvo, E), "attn_v": (kvo, E), "attn_output": (E, qo),
            "ffn_gate": (FD, E), "ffn_up": (FD, E), "ffn_down": (E, FD)}
    for name, (qt, arr) in model.tensors.items():
        if tied and name == "output.weight":
            continue
        a = np.ascontiguousarray(arr)
        if qt == GGML_F32:
            shape = (a.size,)
        else:
            rows, cols = dims[name.split(".")[-2]]
            shape = (cols, rows)
        w.add_tensor(name, a, qt, shape)
    return w


class GgufFile:
    """An open GGUF file (axf_gguf_open); host-only, no GPU needed."""

    def __init__(self, path: str | Path):
        h = C.c_void_p()
        call("axf_gguf_open", str(path).encode(), C.byref(h))
        self.handle = h

    def close(self) -> None:
        if self.handle:
            lib.axf_gguf_close(self.handle)
            self.handle = None

    def __enter__(self) -> "GgufFile":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    @property
    def version(self) -> int:
        return int(lib.axf_gguf_version(self.handle))

    @property
    def alignment(self) -> int:
        return int(lib.axf_gguf_alignment(self.handle))

    @property
    def data_offset(self) -> int:
        return int(lib.axf_gguf_data_offset(self.handle))

    @property
    def n_kv(self) -> int:
        return int(lib.axf_gguf_n_kv(self.handle))

    @property
    def n_tensors(self) -> int:
        return int(lib.axf_gguf_n_tensors(self.handle))

    def kv_type(self, key: str) -> int:
        return int(lib.axf_gguf_kv_type(self.handle, key.encode()))

    def get_u64(self, key: str, default: int = 0) -> int:
        return int(lib.axf_gguf_get_u64(self.handle, key.encode(), default))

    def get_u32(self, key: str, default: int = 0) -> int:
        return int(lib.axf_gguf_get_u32(self.handle, key.encode(), default))

    def get_i32(self, key: str, default: int = 0) -> int:
        return int(lib.axf_gguf_get_i32(self.handle, key.encode(), default))

    def get_f32(self, key: str, default: float = 0.0) -> float:
        return float(lib.axf_gguf_get_f32(self.handle, key.encode(), default))

    def get_bool(self, key: str, default: bool = False) -> bool:
        return bool(lib.axf_gguf_get_bool(self.handle, key.encode(), 1 if default else 0))

    def get_str(self, key: str, default: str | None = None) -> str | None:
        if self.kv_type(key) != STRING:
            return default
        s, n = C.c_char_p(), C.c_size_t()
        call("axf_gguf_get_str", self.handle, key.encode(), C.byref(s), C.byref(n))
        return C.string_at(s, n.value).decode()

    def array_count(self, key: str) -> int:
        return int(lib.axf_gguf_get_array_count(self.handle, key.encode()))

    def array_type(self, key: str) -> int:
        return int(lib.axf_gguf_get_array_type(self.handle, key.encode()))

    def array_strings(self, key: str) -> list[str]:
        out = []
        s, n = C.c_char_p(), C.c_size_t()
        for i in range(self.array_count(key)):
            call("axf_gguf_get_array_str", self.handle, key.encode(), i, C.byref(s), C.byref(n))
            out.append(C.string_at(s, n.value).decode())
        return out

    def array_bytes(self, key: str) -> bytes:
        d, n = C.c_void_p(), C.c_size_t()
        call("axf_gguf_get_array_data", self.handle, key.encode(), C.byref(d), C.byref(n))
        return C.string_at(d, n.value) if n.value else b""

    def tensor(self, i: int | str) -> dict:
        if isinstance(i, str):
            idx = int(lib.axf_gguf_find_tensor(self.handle, i.encode()))
            if idx < 0:
                raise KeyError(i)
            i = idx
        t = GgufTensor()
        call("axf_gguf_tensor_info", self.handle, int(i), C.byref(t))
        return {"name": t.name.decode(), "shape": tuple(t.shape[:t.n_dims]),
                "ggml_type": t.ggml_type, "offset": int(t.offset), "nbytes": int(t.nbytes),
                "data": t.data}

    def tensor_bytes(self, i: int | str) -> bytes:
        t = self.tensor(i)
        if not t["data"]:
            raise ValueError(f"tensor {t['name']}: data lies outside the file")
        return C.string_at(t["data"], t["nbytes"])

    def find_tensor(self, name: str) -> int:
        return int(lib.axf_gguf_find_tensor(self.handle, name.encode()))

    def model_config(self) -> dict:
        c = GgufModelConfig()
        call("axf_gguf_read_model_config", self.handle, C.byref(c))
        d = {name: getattr(c, name) for name, _ in GgufModelConfig._fields_}
        d["arch"] = c.arch.decode()
        return d


def type_nbytes(ggml_type: int, numel: int) -> int:
    return int(lib.axf_gguf_type_nbytes(ggml_type, numel))


def pod_size(tag: int) -> int:
    return int(lib.axf_gguf_pod_size(tag))
