"""ctypes binding of include/axf_hip.h (libaxf_hip.so).

The library is loaded from llm_core_amd/lib/.  There is no fallback: if the
shared object is missing or a symbol is absent, import fails loudly.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libaxf_hip.so"

AXF_OK = 0
AXF_ERR_INVALID_ARG = -1
AXF_ERR_HIP = -2
AXF_ERR_UNSUPPORTED = -3
AXF_ERR_NO_DEVICE = -4
AXF_ERR_STATE = -5

AXF_TYPE_F32 = 0
AXF_TYPE_F16 = 1
AXF_TYPE_Q5_0 = 6
AXF_TYPE_Q8_0 = 8
AXF_TYPE_Q4_K = 12
AXF_TYPE_Q6_K = 14

# axf_llama_get_buffer
AXF_LLAMA_BUF_X = 0
AXF_LLAMA_BUF_QKV = 1
AXF_LLAMA_BUF_ATTN = 2
AXF_LLAMA_BUF_ATTN_Q8 = 3
AXF_LLAMA_BUF_H = 4
AXF_LLAMA_BUF_LOGITS = 5


class AxfError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class LlamaHparams(C.Structure):
    _fields_ = [
        ("n_layer", C.c_int),
        ("n_embd", C.c_int),
        ("n_heads", C.c_int),
        ("n_kv_heads", C.c_int),
        ("ffn_dim", C.c_int),
        ("n_vocab", C.c_int),
        ("n_ctx", C.c_int),
        ("rms_eps", C.c_float),
        ("rope_theta", C.c_float),
        ("qk_norm_order", C.c_int),
    ]


class Sampling(C.Structure):
    _fields_ = [
        ("temperature", C.c_float),
        ("top_k", C.c_int),
        ("top_p", C.c_float),
        ("rep_penalty", C.c_float),
        ("rep_penalty_last_n", C.c_int),
        ("seed", C.c_uint32),
        ("eos_id", C.c_int32),
    ]


class GgufTensor(C.Structure):
    _fields_ = [
        ("name", C.c_char_p),
        ("n_dims", C.c_int),
        ("shape", C.c_int64 * 4),
        ("ggml_type", C.c_int),
        ("offset", C.c_uint64),
        ("nbytes", C.c_uint64),
        ("data", C.c_void_p),
    ]


class GgufModelConfig(C.Structure):
    _fields_ = [
        ("arch", C.c_char * 64),
        ("n_layer", C.c_int),
        ("n_embd", C.c_int),
        ("ffn_dim", C.c_int),
        ("n_heads", C.c_int),
        ("n_kv_heads", C.c_int),
        ("head_dim", C.c_int),
        ("max_seq_len", C.c_int),
        ("n_vocab", C.c_int),
        ("rms_eps", C.c_float),
        ("rope_theta", C.c_float),
        ("rope_scaling_alpha", C.c_float),
        ("weight_type", C.c_int),
        ("bos_id", C.c_int32),
        ("eos_id", C.c_int32),
    ]


vp = C.c_void_p
i32 = C.c_int
i64 = C.c_int64
u64 = C.c_uint64
f32 = C.c_float
sz = C.c_size_t
fp = C.POINTER(C.c_float)

# name -> argtypes (all return int unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "axf_hip_last_error": [],
    "axf_hip_version": [C.POINTER(i32), C.POINTER(i32), C.POINTER(i32)],
    "axf_hip_device_count": [C.POINTER(i32)],
    "axf_hip_create": [i32, C.POINTER(vp)],
    "axf_hip_destroy": [vp],
    "axf_hip_device_name": [vp, C.c_char_p, i32],
    "axf_hip_alloc": [vp, sz, C.POINTER(vp)],
    "axf_hip_free": [vp, vp],
    "axf_hip_memcpy_h2d": [vp, vp, vp, sz],
    "axf_hip_memcpy_d2h": [vp, vp, vp, sz],
    "axf_hip_memcpy_d2d": [vp, vp, vp, sz],
    "axf_hip_sync": [vp],
    "axf_hip_dequant_q4k": [vp, vp, vp, i64],
    "axf_hip_dequant_q6k": [vp, vp, vp, i64],
    "axf_hip_quantize_q8_0": [vp, vp, vp, i32],
    "axf_hip_gemv_q4k_f32": [vp, vp, vp, vp, i32, i32, sz],
    "axf_hip_gemv_q6k_f32": [vp, vp, vp, vp, i32, i32, sz],
    "axf_hip_gemv_q4k_q8": [vp, vp, vp, vp, i32, i32, sz, i32],
    "axf_hip_gemv_q6k_q8": [vp, vp, vp, vp, i32, i32, sz, i32],
    "axf_hip_gemm_q4k_q8": [vp, vp, vp, vp, i32, i32, i32, sz],
    "axf_hip_gemm_q4k_q8_path": [vp, vp, vp, vp, i32, i32, i32, sz, i32],
    "axf_hip_gemm_q4k_q8_noalloc": [vp, vp, vp, vp, i32, i32, i32, sz],
    "axf_hip_gemm_q6k_q8": [vp, vp, vp, vp, i32, i32, i32, sz],
    "axf_hip_gemm_q6k_q8_path": [vp, vp, vp, vp, i32, i32, i32, sz, i32],
    "axf_hip_argmax_f32": [vp, vp, vp, i32],
    "axf_hip_gemv_q8_0w_q8": [vp, vp, vp, vp, i32, i32, sz, i32],
    "axf_hip_gemv_q8_0w_f32": [vp, vp, vp, vp, i32, i32, sz],
    "axf_hip_gemv_q5_0_f32": [vp, vp, vp, vp, i32, i32, sz],
    "axf_hip_gemv_f16_f32": [vp, vp, vp, vp, vp, i32, i32],
    "axf_hip_gemm_misc_f32": [vp, i32, vp, vp, vp, i32, i32, i32, sz, i32],
    "axf_hip_sample": [vp, vp, i32, C.POINTER(Sampling), vp, i32, f32, C.POINTER(C.c_int32)],
    "axf_mt19937": [C.c_uint32, vp, i32],
    "axf_sampling_uniforms": [C.c_uint32, vp, i32],
    "axf_hip_rmsnorm": [vp, vp, vp, vp, vp, i32, f32],
    "axf_rope_table": [vp, vp, i32, f32, i32],
    "axf_hip_rope": [vp, vp, vp, i32, i32, i32, vp, vp],
    "axf_hip_attn_decode": [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32],
    "axf_hip_attn_prefill": [vp, vp, vp, vp, i32, vp, vp, vp, i32, i32, i32, i32, i32, vp, vp,
                             i32],
    "axf_hip_swiglu": [vp, vp, vp, vp, vp, i32],
    "axf_hip_add": [vp, vp, vp, vp, i32],
    "axf_hip_embed": [vp, vp, i32, vp, i32, i32, i32],
    "axf_hip_timer_start": [vp],
    "axf_hip_timer_stop": [vp, C.POINTER(f32)],
    "axf_hip_bench_gemv": [vp, i32, vp, C.POINTER(vp), i32, vp, i32, i32, sz, i32, C.POINTER(f32)],
    "axf_hip_bench_set_eager": [vp, i32],
    "axf_hip_bench_read": [vp, C.POINTER(vp), i32, sz, i32, i32, i32, C.POINTER(f32)],
    "axf_hip_bench_gemm": [vp, i32, vp, C.POINTER(vp), i32, vp, i32, i32, i32, sz, i32, i32,
                           C.POINTER(f32)],
    "axf_synth_normal": [vp, i64, u64, f32, f32],
    "axf_synth_quantize": [i32, vp, vp, i64],
    "axf_synth_weight": [i32, vp, i64, i64, u64, f32],
    "axf_row_bytes": [i32, i64],
    "axf_llama_create": [vp, C.POINTER(LlamaHparams), C.POINTER(vp)],
    "axf_llama_destroy": [vp],
    "axf_llama_set_tensor": [vp, C.c_char_p, i32, vp, sz],
    "axf_llama_load": [vp],
    "axf_llama_load_gguf": [vp, vp],
    "axf_llama_get_hparams": [vp, C.POINTER(LlamaHparams)],
    "axf_llama_from_gguf": [vp, C.c_char_p, i32, C.POINTER(vp)],
    "axf_gguf_open": [C.c_char_p, C.POINTER(vp)],
    "axf_gguf_close": [vp],
    "axf_gguf_version": [vp],
    "axf_gguf_alignment": [vp],
    "axf_gguf_data_offset": [vp],
    "axf_gguf_file_size": [vp],
    "axf_gguf_n_kv": [vp],
    "axf_gguf_n_tensors": [vp],
    "axf_gguf_kv_type": [vp, C.c_char_p],
    "axf_gguf_get_u64": [vp, C.c_char_p, u64],
    "axf_gguf_get_u32": [vp, C.c_char_p, C.c_uint32],
    "axf_gguf_get_i32": [vp, C.c_char_p, C.c_int32],
    "axf_gguf_get_f32": [vp, C.c_char_p, f32],
    "axf_gguf_get_bool": [vp, C.c_char_p, i32],
    "axf_gguf_get_str": [vp, C.c_char_p, C.POINTER(C.c_char_p), C.POINTER(sz)],
    "axf_gguf_get_array_count": [vp, C.c_char_p],
    "axf_gguf_get_array_type": [vp, C.c_char_p],
    "axf_gguf_get_array_str": [vp, C.c_char_p, u64, C.POINTER(C.c_char_p), C.POINTER(sz)],
    "axf_gguf_get_array_data": [vp, C.c_char_p, C.POINTER(vp), C.POINTER(sz)],
    "axf_gguf_tensor_info": [vp, i64, C.POINTER(GgufTensor)],
    "axf_gguf_find_tensor": [vp, C.c_char_p],
    "axf_gguf_type_nbytes": [i32, i64],
    "axf_gguf_pod_size": [i32],
    "axf_gguf_read_model_config": [vp, C.POINTER(GgufModelConfig)],
    "axf_llama_device_bytes": [vp],
    "axf_llama_set_x": [vp, vp],
    "axf_llama_get_x": [vp, vp],
    "axf_llama_set_kv": [vp, i32, vp, vp, i32],
    "axf_llama_fill_kv_random": [vp, i32, u64],
    "axf_llama_get_logits": [vp, vp],
    "axf_llama_forward_layer": [vp, i32, i32],
    "axf_llama_forward_layer_stages": [vp, i32, i32, i32, i32],
    "axf_llama_get_buffer": [vp, i32, vp, sz],
    "axf_llama_get_kv": [vp, i32, vp, vp, i32, i32],
    "axf_llama_forward_token": [vp, i32, i32],
    "axf_llama_generate": [vp, vp, i32, i32, vp, i32],
    "axf_llama_generate_ex": [vp, vp, i32, i32, vp, i32, i32],
    "axf_llama_generate_sampled": [vp, vp, i32, i32, C.POINTER(Sampling), vp, C.POINTER(i32),
                                   i32],
    "axf_llama_forward_batch": [vp, vp, i32, i32],
    "axf_llama_bench_prefill": [vp, i32, i32, C.POINTER(f32)],
    "axf_llama_bench_decode": [vp, i32, i32, i32, C.POINTER(f32)],
    "axf_llama_bench_stage": [vp, i32, i32, i32, C.POINTER(f32)],
}

_RESTYPES = {
    "axf_hip_last_error": C.c_char_p,
    "axf_row_bytes": sz,
    "axf_llama_device_bytes": sz,
    "axf_gguf_version": C.c_uint32,
    "axf_gguf_alignment": u64,
    "axf_gguf_data_offset": u64,
    "axf_gguf_file_size": u64,
    "axf_gguf_n_kv": i64,
    "axf_gguf_n_tensors": i64,
    "axf_gguf_get_u64": u64,
    "axf_gguf_get_u32": C.c_uint32,
    "axf_gguf_get_i32": C.c_int32,
    "axf_gguf_get_f32": f32,
    "axf_gguf_get_array_count": u64,
    "axf_gguf_find_tensor": i64,
    "axf_gguf_type_nbytes": sz,
    "axf_gguf_pod_size": sz,
}


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m llm_core_amd.build` "
            "(there is no CPU fallback for the HIP path)"
        )
    lib = C.CDLL(str(LIB_PATH))
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the symbol is missing
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, C.c_int)
    return lib


lib = _load()


def last_error() -> str:
    msg = lib.axf_hip_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> None:
    if rc != AXF_OK:
        raise AxfError(rc, last_error())


def call(name: str, *args) -> None:
    check(getattr(lib, name)(*args))
