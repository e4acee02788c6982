"""GGUF reader (axf_gguf_*, host code) against the reference's GgufReader
behaviour: its test fixtures (tests/test_gguf_reader.cpp:31-200 builds the same
minimal LLaMA, Qwen2 and Qwen2.5-3B files) and known answers, plus the error
paths of gguf_loader.cpp:84-163.  No GPU needed."""
import math
import struct

import numpy as np
import pytest

from llm_core_amd import gguf as G
from llm_core_amd._ffi import AxfError


def minimal_llama() -> G.GGUFWriter:
    """make_minimal_gguf of the reference test: 9 KV pairs, one F32 [4, 4] tensor."""
    w = G.GGUFWriter()
    w.add("general.architecture", G.STRING, "llama")
    w.add("llama.block_count", G.U64, 4)
    w.add("llama.embedding_length", G.U64, 32)
    w.add("llama.feed_forward_length", G.U64, 64)
    w.add("llama.attention.head_count", G.U64, 4)
    w.add("llama.rope.freq_base", G.F32, 500000.0)
    w.add("tokenizer.ggml.bos_token_id", G.U32, 128000)
    w.add("tokenizer.ggml.eos_token_id", G.U32, 128001)
    w.add_array("tokenizer.ggml.tokens", G.STRING, ["<unk>", "<bos>", "<eos>", "hello", "world"])
    w.add_tensor("weight.0", np.arange(16, dtype=np.float32), G.GGML_F32, (4, 4))
    return w


def qwen2(layers=24, embd=896, ffn=4864, heads=14, kv=2) -> G.GGUFWriter:
    w = G.GGUFWriter()
    w.add("general.architecture", G.STRING, "qwen2")
    w.add("qwen2.block_count", G.U64, layers)
    w.add("qwen2.embedding_length", G.U64, embd)
    w.add("qwen2.feed_forward_length", G.U64, ffn)
    w.add("qwen2.attention.head_count", G.U64, heads)
    w.add("qwen2.attention.head_count_kv", G.U64, kv)
    w.add("qwen2.context_length", G.U64, 32768)
    w.add("qwen2.attention.layer_norm_rms_epsilon", G.F32, 1e-6)
    w.add("qwen2.rope.freq_base", G.F32, 1000000.0)
    w.add("tokenizer.ggml.bos_token_id", G.U32, 151643)
    w.add("tokenizer.ggml.eos_token_id", G.U32, 151645)
    w.add_array("tokenizer.ggml.tokens", G.STRING,
                ["h", "e", "l", "o", "he", "hel", "hell", "hello", "<|im_start|>", "<|im_end|>"])
    w.add_array("tokenizer.ggml.merges", G.STRING, ["h e", "he l", "hel l", "hell o"])
    w.add_array("tokenizer.ggml.token_type", G.I32, [1, 1, 1, 1, 1, 1, 1, 1, 3, 3])
    w.add_tensor("weight.0", np.arange(16, dtype=np.float32), G.GGML_F32, (4, 4))
    return w


def open_bytes(tmp_path, data: bytes, name="t.gguf") -> G.GgufFile:
    p = tmp_path / name
    p.write_bytes(data)
    return G.GgufFile(p)


def open_error(tmp_path, data: bytes) -> str:
    with pytest.raises(AxfError) as e:
        open_bytes(tmp_path, data)
    return str(e.value)


def test_minimal_header_tensor_and_data(tmp_path):
    with open_bytes(tmp_path, minimal_llama().to_bytes()) as f:
        assert f.version == 3 and f.alignment == 32 and f.n_kv == 9 and f.n_tensors == 1
        assert f.data_offset % 32 == 0
        t = f.tensor(0)
        assert (t["name"], t["shape"], t["ggml_type"], t["offset"], t["nbytes"]) == \
            ("weight.0", (4, 4), 0, 0, 64)
        assert f.find_tensor("weight.0") == 0 and f.find_tensor("nope") == -1
        np.testing.assert_array_equal(np.frombuffer(f.tensor_bytes("weight.0"), np.float32),
                                      np.arange(16, dtype=np.float32))


def test_minimal_model_config(tmp_path):
    """Engine::from_gguf reads LLaMA hyperparams (the reference's test: 4 layers,
    hidden 32, FFN 64, 4 heads, head_dim 8, theta 500000); absent keys take
    the defaults (KV heads = heads, context 4096, eps 1e-5)."""
    with open_bytes(tmp_path, minimal_llama().to_bytes()) as f:
        c = f.model_config()
    assert c["arch"] == "llama"
    assert (c["n_layer"], c["n_embd"], c["ffn_dim"], c["n_heads"], c["n_kv_heads"],
            c["head_dim"], c["max_seq_len"], c["n_vocab"]) == (4, 32, 64, 4, 4, 8, 4096, 5)
    assert c["rope_theta"] == pytest.approx(500000.0, rel=1e-5)
    assert c["rms_eps"] == pytest.approx(1e-5, rel=1e-5)
    assert (c["bos_id"], c["eos_id"], c["weight_type"]) == (128000, 128001, 0)


def test_qwen2_config_and_tokenizer_arrays(tmp_path):
    with open_bytes(tmp_path, qwen2().to_bytes()) as f:
        c = f.model_config()
        assert c["arch"] == "qwen2"
        assert (c["n_layer"], c["n_embd"], c["ffn_dim"], c["n_heads"], c["n_kv_heads"],
                c["head_dim"], c["max_seq_len"], c["n_vocab"]) == (24, 896, 4864, 14, 2, 64,
                                                                   32768, 10)
        assert c["rope_theta"] == pytest.approx(1e6, rel=1e-5)
        assert c["rms_eps"] == pytest.approx(1e-6, rel=1e-5)
        assert f.array_strings("tokenizer.ggml.merges") == ["h e", "he l", "hel l", "hell o"]
        assert f.array_type("tokenizer.ggml.token_type") == G.I32
        assert list(np.frombuffer(f.array_bytes("tokenizer.ggml.token_type"), np.int32)) == \
            [1] * 8 + [3, 3]
        assert f.array_strings("tokenizer.ggml.tokens")[8] == "<|im_start|>"


def test_qwen25_3b_config(tmp_path):
    with open_bytes(tmp_path, qwen2(36, 2048, 11008, 16, 2).to_bytes()) as f:
        c = f.model_config()
    assert (c["n_layer"], c["n_embd"], c["ffn_dim"], c["n_heads"], c["n_kv_heads"],
            c["head_dim"], c["n_vocab"]) == (36, 2048, 11008, 16, 2, 128, 10)


def test_hunyuan_dense_theta_scaling(tmp_path):
    """rope theta *= alpha^(hd/(hd-2)) for hunyuan-dense (engine.cpp:100-103)."""
    w = G.GGUFWriter()
    w.add("general.architecture", G.STRING, "hunyuan-dense")
    w.add("hunyuan-dense.embedding_length", G.U64, 2048)
    w.add("hunyuan-dense.attention.head_count", G.U64, 16)
    w.add("hunyuan-dense.rope.freq_base", G.F32, 500000.0)
    w.add("hunyuan-dense.rope.scaling.alpha", G.F32, 32.0)
    with open_bytes(tmp_path, w.to_bytes()) as f:
        c = f.model_config()
    assert c["head_dim"] == 128 and c["rope_scaling_alpha"] == 32.0
    assert c["rope_theta"] == pytest.approx(500000.0 * 32.0 ** (128 / 126), rel=1e-5)


def test_type_tables():
    """Known answers of the reference's dtype tests (test_gguf_reader.cpp:201-250)."""
    cases = [(0, 16, 64), (1, 32, 64), (8, 32, 34), (8, 64, 68), (2, 32, 18), (2, 64, 36),
             (6, 32, 22), (6, 64, 44), (12, 256, 144), (12, 512, 288), (10, 256, 84),
             (0, 0, 0), (14, 256, 210), (14, 512, 420), (30, 8, 16), (99, 256, 0),
             (8, 33, 68), (12, 257, 288)]  # partial blocks round up
    for t, n, want in cases:
        assert G.type_nbytes(t, n) == want, (t, n)
    assert [G.pod_size(k) for k in range(13)] == [1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8]
    assert G.pod_size(13) == 0


def test_version_2_parses(tmp_path):
    w = minimal_llama()
    w.version = 2
    with open_bytes(tmp_path, w.to_bytes()) as f:
        assert f.version == 2 and f.model_config()["n_layer"] == 4


@pytest.mark.parametrize("version", [0, 1, 4, 0xFFFFFFFF])
def test_unsupported_version(tmp_path, version):
    w = minimal_llama()
    w.version = version
    assert f"unsupported GGUF version {version} (supported: 2, 3)" in open_error(tmp_path, w.to_bytes())


def test_bad_magic_and_tiny_file(tmp_path):
    w = minimal_llama()
    w.magic = b"GGML"
    assert "invalid magic (not a GGUF file)" in open_error(tmp_path, w.to_bytes())
    assert "file too small" in open_error(tmp_path, b"GGUF\x03\0\0\0")
    with pytest.raises(AxfError, match="cannot open"):
        G.GgufFile(tmp_path / "missing.gguf")


def test_every_truncation_fails_cleanly(tmp_path):
    """Every prefix of the header and metadata is a clean error, never a crash;
    a file cut inside the data blob still parses (the blob is not read at open)."""
    w = minimal_llama()
    data = w.to_bytes()
    info_end = 24 + sum(map(len, w.kv)) + sum(map(len, w.infos))  # before the padding
    for n in range(16, info_end):
        msg = open_error(tmp_path, data[:n])
        assert "truncated" in msg, (n, msg)
    with open_bytes(tmp_path, data[:info_end]) as f:  # padding is skipped, not read
        assert f.n_tensors == 1 and f.tensor(0)["data"] is None
    with open_bytes(tmp_path, data[:-8]) as f:
        assert f.tensor(0)["data"] is None  # its 64 bytes leave the file
        with pytest.raises(ValueError):
            f.tensor_bytes(0)


def test_negative_counts(tmp_path):
    w = minimal_llama()
    assert "negative tensor/kv counts" in open_error(tmp_path, w.to_bytes(n_tensors=-1))
    assert "negative tensor/kv counts" in open_error(tmp_path, w.to_bytes(n_kv=-5))


def test_bad_tensor_infos(tmp_path):
    w = G.GGUFWriter()
    w.raw_tensor_info(G._str("t5") + struct.pack("<I", 5) + struct.pack("<5q", 1, 1, 1, 1, 1) +
                      struct.pack("<iQ", 0, 0))
    assert "tensor 't5' has more than 4 dimensions (5)" in open_error(tmp_path, w.to_bytes())
    w = G.GGUFWriter()
    w.raw_tensor_info(G._str("tn") + struct.pack("<I", 2) + struct.pack("<2q", 4, -1) +
                      struct.pack("<iQ", 0, 0))
    assert "tensor 'tn' has negative dimension" in open_error(tmp_path, w.to_bytes())


def test_bad_kv_types(tmp_path):
    w = G.GGUFWriter().raw_kv(G._str("k") + struct.pack("<i", 13) + b"\0" * 8)
    assert "unknown KV type tag 13" in open_error(tmp_path, w.to_bytes())
    w = G.GGUFWriter().raw_kv(G._str("k") + struct.pack("<iiQ", G.ARRAY, G.ARRAY, 1) + b"\0" * 16)
    assert "nested ARRAY or unknown type in array" in open_error(tmp_path, w.to_bytes())
    # an array count far beyond the file is a truncation, not an allocation
    w = G.GGUFWriter().raw_kv(G._str("k") + struct.pack("<iiQ", G.ARRAY, G.U32, 1 << 60))
    assert "truncated" in open_error(tmp_path, w.to_bytes())
    w = G.GGUFWriter().raw_kv(G._str("k") + struct.pack("<iiQ", G.ARRAY, G.STRING, 1 << 60))
    assert "truncated" in open_error(tmp_path, w.to_bytes())


def test_alignment_key(tmp_path):
    """general.alignment is honoured only as a u32 (gguf_loader.cpp:113-119);
    the data blob and every tensor offset follow it."""
    w = minimal_llama()
    w.alignment = 64
    w.add("general.alignment", G.U32, 64)
    w.add_tensor("weight.1", np.ones(3, np.float32), G.GGML_F32, (3,))
    with open_bytes(tmp_path, w.to_bytes()) as f:
        assert f.alignment == 64 and f.data_offset % 64 == 0
        assert f.tensor("weight.1")["offset"] == 64
        assert np.frombuffer(f.tensor_bytes("weight.1"), np.float32).tolist() == [1.0] * 3
    w = minimal_llama().add("general.alignment", G.U64, 64)
    with open_bytes(tmp_path, w.to_bytes()) as f:
        assert f.alignment == 32
    w = minimal_llama().add("general.alignment", G.U32, 0)
    assert "general.alignment must be non-zero" in open_error(tmp_path, w.to_bytes())


def test_typed_accessors(tmp_path):
    """The reference's coercions: get_u64/u32 from any integer type, get_i32 from
    32/64-bit integers only, get_f32 from f32 or f64, get_bool from bool only;
    the default otherwise."""
    w = G.GGUFWriter()
    for tag, v in [(G.U8, 200), (G.I8, -3), (G.U16, 60000), (G.I16, -7), (G.U32, 4000000000),
                   (G.I32, -9), (G.U64, 1 << 40), (G.I64, -(1 << 33)), (G.F32, 1.5),
                   (G.F64, 2.25), (G.BOOL, True)]:
        w.add(f"k{tag}", tag, v)
    w.add("s", G.STRING, "text")
    w.add("first", G.U32, 1).add("first", G.U32, 2)  # duplicate key: the first is kept
    with open_bytes(tmp_path, w.to_bytes()) as f:
        assert f.get_u64(f"k{G.U8}") == 200 and f.get_u64(f"k{G.U16}") == 60000
        assert f.get_u64(f"k{G.I8}") == (1 << 64) - 3
        assert f.get_u64(f"k{G.U64}") == 1 << 40 and f.get_u32(f"k{G.U64}") == 0
        assert f.get_i32(f"k{G.I32}") == -9 and f.get_i32(f"k{G.U32}") == 4000000000 - (1 << 32)
        assert f.get_i32(f"k{G.U16}", 77) == 77  # 16-bit values are not converted
        assert f.get_f32(f"k{G.F32}") == 1.5 and f.get_f32(f"k{G.F64}") == 2.25
        assert f.get_f32(f"k{G.U32}", -1.0) == -1.0
        assert f.get_bool(f"k{G.BOOL}") is True and f.get_bool(f"k{G.U8}", False) is False
        assert f.get_str("s") == "text" and f.get_str(f"k{G.U8}") is None
        assert f.get_u64("missing", 123) == 123 and f.kv_type("missing") == -1
        assert f.kv_type("s") == G.STRING and f.kv_type(f"k{G.F64}") == G.F64
        assert f.get_u32("first") == 1


def test_synthetic_model_round_trip(tmp_path):
    """llama_gguf writes every tensor of a synthetic model unchanged, with GGML
    shapes and sizes the reader recomputes from the type."""
    from llm_core_amd.model import Hparams, SynthLlama

    hp = Hparams(n_layer=2, n_embd=512, n_heads=8, n_kv_heads=4, ffn_dim=1024, n_vocab=300,
                 n_ctx=64)
    m = SynthLlama(hp, seed=2, norm_std=0.1, with_bias=True)
    p = G.llama_gguf(m, arch="qwen2").write(tmp_path / "m.gguf")
    with G.GgufFile(p) as f:
        assert f.n_tensors == len(m.tensors)
        c = f.model_config()
        assert (c["arch"], c["n_layer"], c["n_embd"], c["n_heads"], c["n_kv_heads"], c["ffn_dim"],
                c["n_vocab"], c["max_seq_len"]) == ("qwen2", 2, 512, 8, 4, 1024, 300, 64)
        for name, (qt, arr) in m.tensors.items():
            t = f.tensor(name)
            assert t["ggml_type"] == qt and t["offset"] % 32 == 0
            assert t["nbytes"] == arr.nbytes == math.prod(t["shape"]) // {0: 1, 12: 256, 14: 256}[qt] \
                * {0: 4, 12: 144, 14: 210}[qt]
            assert f.tensor_bytes(name) == np.ascontiguousarray(arr).tobytes()
        assert f.tensor("blk.1.ffn_down.weight")["shape"] == (1024, 512)
