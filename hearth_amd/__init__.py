"""hearth_amd — MI355X (gfx950) batch-1 decode path for Hearth-style quantized LLMs.

The compute lives in ``libhearth_hip.so`` (HIP kernels + a C ABI declared in
``include/hearth_hip.h``); this package is a thin ctypes binding over that ABI,
the same surface a Rust FFI crate in hearth-llm would bind.  There is no CPU
fallback: importing the binding without the built library raises.
"""
from .lib import (  # noqa: F401
    HHError,
    Ctx,
    Model,
    Gguf,
    ModelConfig,
    CONFIGS,
    GGML_F32,
    GGML_F16,
    GGML_Q8_0,
    GGML_Q1_0,
    GGML_Q2_0,
    GGML_Q1_0_G128,
    GGML_PQ2_0,
    GGML_PTQ1_0,
    lib_path,
    load_library,
    row_bytes,
)
