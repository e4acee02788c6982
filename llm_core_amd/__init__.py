"""llm_core_amd — MI355X (gfx950) native quantized decode path for GGUF
Q4_K / Q6_K models (the hot path of songqiuyu/llm_core "AxonForge").

    llm_core_amd.build   build libaxf_hip.so in-tree
    llm_core_amd.hip     device context, buffers and C-ABI kernel calls
    llm_core_amd.model   synthetic Q4_K_M LLaMA models and the device decoder
"""

__version__ = "0.1.0"
