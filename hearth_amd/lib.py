"""ctypes binding of include/hearth_hip.h.

Mirrors the reference's operator/model surface:
  * ``Ctx`` — device context (hearth_compute::GpuCompute::new, lib.rs:126), operator
    entry points on device buffers (torch tensors on cuda, passed by pointer);
  * ``Model`` — weights in HBM + KV/recurrent state + the device token loop
    (LlamaModel::forward / generate_text, mod.rs:451-860, :2718-3012;
    Qwen35Core::forward / generate_text, qwen35.rs:1028-1236, :1654-1804).
Errors come back as ``HHError`` carrying the library's status and message, the
counterpart of the reference's ``Result<_, String>``.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import os
from typing import Optional, Sequence

import numpy as np

GGML_F32, GGML_F16, GGML_Q8_0 = 0, 1, 8
GGML_Q1_0, GGML_Q2_0, GGML_Q1_0_G128, GGML_PQ2_0, GGML_PTQ1_0 = 41, 42, 43, 142, 143

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB: Optional[C.CDLL] = None


def lib_path() -> str:
    return os.path.join(_HERE, "libhearth_hip.so")


def row_bytes(t: int, n: int) -> int:
    """Bytes of one row of n elements (ggml.rs:105-171)."""
    if t == GGML_F32:
        return 4 * n
    if t == GGML_F16:
        return 2 * n
    if t == GGML_Q8_0:
        return n // 32 * 34
    if t in (GGML_Q1_0, GGML_Q1_0_G128):
        return n // 128 * 18
    if t in (GGML_Q2_0, GGML_PQ2_0):
        return n // 128 * 34
    if t == GGML_PTQ1_0:
        return n // 128 * 28
    raise ValueError(f"unknown ggml type {t}")


# hh_status (include/hearth_hip.h)
HH_OK, HH_ERR_INVALID, HH_ERR_DTYPE, HH_ERR_DIM, HH_ERR_OOM, HH_ERR_HIP, HH_ERR_NOT_FOUND, HH_ERR_RANGE, \
    HH_ERR_CANCELLED = range(9)


class HHError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"hearth_hip status {status}: {msg}")
        self.status = status


class ModelConfigC(C.Structure):
    _fields_ = [
        ("arch", C.c_int), ("d_model", C.c_int), ("n_layers", C.c_int), ("n_heads", C.c_int),
        ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("d_ffn", C.c_int), ("vocab", C.c_int),
        ("eps", C.c_float), ("rope_theta", C.c_float), ("rope_dim", C.c_int), ("max_seq", C.c_int),
        ("wtype", C.c_int), ("head_type", C.c_int), ("qk_norm", C.c_int),
        ("full_attn_interval", C.c_int), ("ssm_n_k_heads", C.c_int), ("ssm_n_v_heads", C.c_int),
        ("ssm_head_dim", C.c_int), ("ssm_conv_kernel", C.c_int), ("attn_out_gate", C.c_int),
        ("kv_type", C.c_int), ("had_block", C.c_int), ("had_flags", C.c_int),
    ]


@dataclasses.dataclass
class ModelConfig:
    """hh_model_config / ho_config (the BASELINE.json model geometries)."""
    arch: int = 0
    d_model: int = 2048
    n_layers: int = 28
    n_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    d_ffn: int = 6144
    vocab: int = 151936
    eps: float = 1e-6
    rope_theta: float = 1e6
    rope_dim: int = 0
    max_seq: int = 4096
    wtype: int = GGML_Q1_0
    head_type: int = GGML_Q8_0
    qk_norm: int = 1
    full_attn_interval: int = 4
    ssm_n_k_heads: int = 0
    ssm_n_v_heads: int = 0
    ssm_head_dim: int = 128
    ssm_conv_kernel: int = 4
    attn_out_gate: int = 0
    kv_type: int = 0        # 0 = f32 KV cache, 8 = Q8_0 rows
    had_block: int = 0      # qwen35 Hadamard fold block size (0 = no fold)
    had_flags: int = 0      # 1 = latent token_embd (R^-1 after lookup), 2 = tied output

    def to_c(self) -> ModelConfigC:
        return ModelConfigC(*[getattr(self, f[0]) for f in ModelConfigC._fields_])

    def replace(self, **kw) -> "ModelConfig":
        return dataclasses.replace(self, **kw)


# BASELINE.json configs.  Head/embedding Q8_0 everywhere.  The 9B/27B hybrids use
# partial RoPE over 64 of 256 dims; the 27B attention/GDN head counts are not in
# BASELINE and are stated here (24 q / 4 kv x 256; GDN 16 k / 32 v x 128).
CONFIGS = {
    "1.7b-q1": ModelConfig(),
    "8b-q2": ModelConfig(d_model=4096, n_layers=36, n_heads=32, n_kv_heads=8, head_dim=128,
                         d_ffn=12288, wtype=GGML_Q2_0, max_seq=2304),
    "9b-hybrid-q2": ModelConfig(arch=1, d_model=4096, n_layers=32, n_heads=16, n_kv_heads=4,
                                head_dim=256, rope_dim=64, d_ffn=12288, vocab=248320,
                                wtype=GGML_Q2_0, max_seq=1024, full_attn_interval=4,
                                ssm_n_k_heads=16, ssm_n_v_heads=32, ssm_head_dim=128,
                                ssm_conv_kernel=4, attn_out_gate=1),
    "27b-hybrid-pq2": ModelConfig(arch=1, d_model=5120, n_layers=64, n_heads=24, n_kv_heads=4,
                                  head_dim=256, rope_dim=64, d_ffn=17408, vocab=248320,
                                  wtype=GGML_PQ2_0, max_seq=8192 + 64, full_attn_interval=4,
                                  ssm_n_k_heads=16, ssm_n_v_heads=32, ssm_head_dim=128,
                                  ssm_conv_kernel=4, attn_out_gate=1),
}

_EXPORTS = {
    "hh_last_error": (C.c_char_p, []),
    "hh_version": (C.c_char_p, []),
    "hh_ctx_create": (C.c_int, [C.c_int, C.POINTER(C.c_void_p)]),
    "hh_ctx_destroy": (C.c_int, [C.c_void_p]),
    "hh_ctx_synchronize": (C.c_int, [C.c_void_p]),
    "hh_malloc": (C.c_int, [C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p)]),
    "hh_free": (C.c_int, [C.c_void_p, C.c_void_p]),
    "hh_memcpy_h2d": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    "hh_memcpy_d2h": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    "hh_memset": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_size_t]),
    "hh_ctx_event_record": (C.c_int, [C.c_void_p, C.c_int]),
    "hh_ctx_event_elapsed": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_float)]),
    "hh_quantize_q8_0": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]),
    "hh_dequantize": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int64, C.c_void_p]),
    "hh_gemv_q8": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p]),
    "hh_gemm_q8": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int64, C.c_int64, C.c_void_p, C.c_int64,
                             C.c_void_p]),
    "hh_rms_norm": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_float, C.c_int64, C.c_int64, C.c_void_p]),
    "hh_rope": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int]),
    "hh_attention": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                C.c_int, C.c_int, C.c_void_p]),
    "hh_attention_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                C.c_int, C.c_int, C.c_void_p]),
    "hh_attention_prefill": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "hh_argmax": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_int64, C.c_float, C.c_int,
                             C.c_void_p]),
    "hh_model_create": (C.c_int, [C.c_void_p, C.POINTER(ModelConfigC), C.POINTER(C.c_void_p)]),
    "hh_model_destroy": (C.c_int, [C.c_void_p]),
    "hh_model_upload_tensor": (C.c_int, [C.c_void_p, C.c_char_p, C.c_int, C.c_int64, C.c_int64, C.c_void_p,
                                          C.c_size_t]),
    "hh_model_download_tensor": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_size_t]),
    "hh_model_tensor_count": (C.c_int, [C.c_void_p]),
    "hh_model_tensor_info": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_char_p), C.POINTER(C.c_int),
                                        C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.POINTER(C.c_size_t)]),
    "hh_model_synthesize": (C.c_int, [C.c_void_p, C.c_uint64]),
    "hh_model_set_hadamard_signs": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p]),
    "hh_model_download_state": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t]),
    "hh_model_reset": (C.c_int, [C.c_void_p]),
    "hh_model_prefill_kv_synthetic": (C.c_int, [C.c_void_p, C.c_uint64, C.c_int]),
    "hh_model_set_cancel": (C.c_int, [C.c_void_p, C.c_int]),
    "hh_model_forward": (C.c_int, [C.c_void_p, C.c_uint32, C.c_int, C.c_void_p, C.POINTER(C.c_uint32)]),
    "hh_model_generate": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_float, C.c_void_p,
                                     C.c_void_p]),
    "hh_model_last_decode_ms": (C.c_int, [C.c_void_p, C.POINTER(C.c_double)]),
    "hh_model_time_stages": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int]),
    "hh_read_bandwidth": (C.c_int, [C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]),
    "hh_model_prefill": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int]),
    "hh_model_last_prefill_ms": (C.c_int, [C.c_void_p, C.POINTER(C.c_double)]),
    "hh_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "hh_gguf_close": (C.c_int, [C.c_void_p]),
    "hh_gguf_header": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "hh_gguf_tensor_count": (C.c_int, [C.c_void_p]),
    "hh_gguf_tensor_info": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_char_p), C.POINTER(C.c_int),
                                       C.POINTER(C.c_int), C.POINTER(C.c_int64), C.POINTER(C.c_uint64),
                                       C.POINTER(C.c_uint64)]),
    "hh_gguf_tensor_data": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_void_p)]),
    "hh_gguf_meta_u32": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_uint32)]),
    "hh_gguf_meta_f32": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_float)]),
    "hh_gguf_meta_str": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_char_p)]),
    "hh_gguf_meta_array_len": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_uint64)]),
    "hh_gguf_model_config": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(ModelConfigC)]),
    "hh_model_load_gguf": (C.c_int, [C.c_void_p, C.c_char_p, C.c_int, C.POINTER(C.c_void_p)]),
}


def exported_symbols() -> Sequence[str]:
    return list(_EXPORTS)


def load_library() -> C.CDLL:
    """Load libhearth_hip.so; raise if it has not been built (no fallback path)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    p = lib_path()
    if not os.path.exists(p):
        raise ImportError(f"{p} is missing: build it with `python -m hearth_amd.build` "
                          "(or __graft_entry__.build()); there is no CPU fallback")
    lib = C.CDLL(p)
    for name, (res, args) in _EXPORTS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def _check(rc: int) -> None:
    if rc != 0:
        msg = load_library().hh_last_error().decode(errors="replace")
        raise HHError(rc, msg)


def _ptr(x) -> int:
    """Device pointer of a torch tensor (or an int address).

    The library runs on its own stream, so torch's pending work on a tensor
    (an async fill or copy on torch's current stream) is waited for first."""
    if isinstance(x, int):
        return x
    if x is None:
        return 0
    if getattr(x, "is_cuda", False):
        import torch
        torch.cuda.current_stream(x.device).synchronize()
    return x.data_ptr()


class Ctx:
    """One device context with its own HIP stream.

    Operator calls are asynchronous on that stream; torch work queued on a
    tensor before a call is waited for, but reading a result with torch needs
    ctx.sync() (or torch.cuda.synchronize()) first."""

    def __init__(self, device: int = 0):
        import weakref
        self.lib = load_library()
        h = C.c_void_p()
        _check(self.lib.hh_ctx_create(device, C.byref(h)))
        self.h = h
        self._models = weakref.WeakSet()

    def close(self) -> None:
        """Destroy the context; models created on it are destroyed first."""
        if self.h:
            for m in list(self._models):
                m.close()
            self.lib.hh_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sync(self) -> None:
        _check(self.lib.hh_ctx_synchronize(self.h))

    def event(self, slot: int) -> None:
        _check(self.lib.hh_ctx_event_record(self.h, slot))

    def elapsed_ms(self, a: int, b: int) -> float:
        v = C.c_float()
        _check(self.lib.hh_ctx_event_elapsed(self.h, a, b, C.byref(v)))
        return v.value

    # ---- operators on device tensors (torch cuda tensors or raw addresses) ----
    def quantize_q8_0(self, x, n: int, out) -> None:
        _check(self.lib.hh_quantize_q8_0(self.h, _ptr(x), n, _ptr(out)))

    def dequantize(self, ggml_type: int, w, n: int, out) -> None:
        _check(self.lib.hh_dequantize(self.h, ggml_type, _ptr(w), n, _ptr(out)))

    def gemv_q8(self, ggml_type: int, w, n_rows: int, n_cols: int, x_q8, y) -> None:
        _check(self.lib.hh_gemv_q8(self.h, ggml_type, _ptr(w), n_rows, n_cols, _ptr(x_q8), _ptr(y)))

    def gemm_q8(self, ggml_type: int, w, n_rows: int, n_cols: int, x_q8, seq_len: int, out) -> None:
        """Batched GEMM (prefill): out[s*n_rows + r] for seq_len Q8_0 token rows."""
        _check(self.lib.hh_gemm_q8(self.h, ggml_type, _ptr(w), n_rows, n_cols, _ptr(x_q8), seq_len, _ptr(out)))

    def rms_norm(self, x, w, eps: float, rows: int, n: int, out) -> None:
        _check(self.lib.hh_rms_norm(self.h, _ptr(x), _ptr(w), eps, rows, n, _ptr(out)))

    def rope(self, x, n_heads: int, head_dim: int, rope_dim: int, table, max_seq: int, pos: int) -> None:
        _check(self.lib.hh_rope(self.h, _ptr(x), n_heads, head_dim, rope_dim, _ptr(table), max_seq, pos))

    def attention(self, q, k, v, n_heads, n_kv, head_dim, max_seq, seq_len, out) -> None:
        _check(self.lib.hh_attention(self.h, _ptr(q), _ptr(k), _ptr(v), n_heads, n_kv, head_dim, max_seq,
                                     seq_len, _ptr(out)))

    def attention_noalloc(self, q, k, v, n_heads, n_kv, head_dim, max_seq, seq_len, out) -> None:
        """hh_attention with the partials in the library's fixed per-GPU scratch (no allocation)."""
        _check(self.lib.hh_attention_noalloc(self.h, _ptr(q), _ptr(k), _ptr(v), n_heads, n_kv, head_dim, max_seq,
                                             seq_len, _ptr(out)))

    def attention_prefill(self, q, k, v, n_heads, n_kv, head_dim, max_seq, pos0, n_tokens, mode, out) -> None:
        """Causal attention of n_tokens prompt tokens at positions pos0.. (mode 0:
        the split/merge kernels, 1: the fp32-MFMA flash form)."""
        _check(self.lib.hh_attention_prefill(self.h, _ptr(q), _ptr(k), _ptr(v), n_heads, n_kv, head_dim, max_seq,
                                             pos0, n_tokens, mode, _ptr(out)))

    def argmax(self, logits, n: int, past, n_past: int, pen: float, rule: int, out) -> None:
        _check(self.lib.hh_argmax(self.h, _ptr(logits), n, _ptr(past), n_past, pen, rule, _ptr(out)))


class Gguf:
    """A parsed GGUF file (hh_gguf_*): header, metadata, tensor table.  Host only."""

    def __init__(self, path: str, lib: Optional[C.CDLL] = None):
        self.lib = lib or load_library()
        h = C.c_void_p()
        _check(self.lib.hh_gguf_open(os.fsencode(path), C.byref(h)))
        self.h = h

    def close(self) -> None:
        if self.h:
            self.lib.hh_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def header(self):
        v, off, al = C.c_uint32(), C.c_uint64(), C.c_uint64()
        _check(self.lib.hh_gguf_header(self.h, C.byref(v), C.byref(off), C.byref(al)))
        return v.value, off.value, al.value

    def tensors(self):
        out = []
        for i in range(self.lib.hh_gguf_tensor_count(self.h)):
            name, t, nd = C.c_char_p(), C.c_int(), C.c_int()
            shape = (C.c_int64 * 4)()
            off, nb = C.c_uint64(), C.c_uint64()
            _check(self.lib.hh_gguf_tensor_info(self.h, i, C.byref(name), C.byref(t), C.byref(nd), shape,
                                                C.byref(off), C.byref(nb)))
            out.append(dict(name=name.value.decode(), type=t.value, shape=tuple(shape[:nd.value]),
                            offset=off.value, nbytes=nb.value))
        return out

    def tensor_bytes(self, index: int, nbytes: int) -> bytes:
        p = C.c_void_p()
        _check(self.lib.hh_gguf_tensor_data(self.h, index, C.byref(p)))
        return C.string_at(p, nbytes)

    def meta_u32(self, key: str) -> int:
        v = C.c_uint32()
        _check(self.lib.hh_gguf_meta_u32(self.h, key.encode(), C.byref(v)))
        return v.value

    def meta_f32(self, key: str) -> float:
        v = C.c_float()
        _check(self.lib.hh_gguf_meta_f32(self.h, key.encode(), C.byref(v)))
        return v.value

    def meta_str(self, key: str) -> str:
        v = C.c_char_p()
        _check(self.lib.hh_gguf_meta_str(self.h, key.encode(), C.byref(v)))
        return v.value.decode()

    def meta_array_len(self, key: str) -> int:
        v = C.c_uint64()
        _check(self.lib.hh_gguf_meta_array_len(self.h, key.encode(), C.byref(v)))
        return v.value

    def model_config(self, ctx_cap: int = 0) -> "ModelConfig":
        c = ModelConfigC()
        _check(self.lib.hh_gguf_model_config(self.h, ctx_cap, C.byref(c)))
        return ModelConfig(**{f[0]: getattr(c, f[0]) for f in ModelConfigC._fields_})


class Model:
    """A model resident in HBM; weights synthesized on device or uploaded."""

    def __init__(self, ctx: Ctx, cfg: ModelConfig):
        self.ctx = ctx
        self.cfg = cfg
        self.lib = ctx.lib
        self._c = cfg.to_c()
        h = C.c_void_p()
        _check(self.lib.hh_model_create(ctx.h, C.byref(self._c), C.byref(h)))
        self.h = h
        ctx._models.add(self)

    @classmethod
    def from_gguf(cls, ctx: Ctx, path: str, ctx_cap: int = 0) -> "Model":
        """hh_model_load_gguf: configuration derived from the file's metadata,
        every tensor uploaded from the mapping (LlamaModel::load, mod.rs:103-150)."""
        with Gguf(path, ctx.lib) as g:
            cfg = g.model_config(ctx_cap)
        self = cls.__new__(cls)
        self.ctx, self.cfg, self.lib = ctx, cfg, ctx.lib
        self._c = cfg.to_c()
        h = C.c_void_p()
        _check(self.lib.hh_model_load_gguf(ctx.h, os.fsencode(path), ctx_cap, C.byref(h)))
        self.h = h
        ctx._models.add(self)
        return self

    def close(self) -> None:
        if self.h and self.ctx.h:
            self.lib.hh_model_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self):
        out = []
        for i in range(self.lib.hh_model_tensor_count(self.h)):
            name = C.c_char_p()
            t = C.c_int()
            ne0 = C.c_int64()
            ne1 = C.c_int64()
            nb = C.c_size_t()
            _check(self.lib.hh_model_tensor_info(self.h, i, C.byref(name), C.byref(t), C.byref(ne0),
                                                 C.byref(ne1), C.byref(nb)))
            out.append((name.value.decode(), t.value, ne0.value, ne1.value, nb.value))
        return out

    def synthesize(self, seed: int) -> None:
        _check(self.lib.hh_model_synthesize(self.h, seed))

    def reset(self) -> None:
        _check(self.lib.hh_model_reset(self.h))

    def prefill_kv_synthetic(self, seed: int, n_pos: int) -> None:
        _check(self.lib.hh_model_prefill_kv_synthetic(self.h, seed, n_pos))

    def download_state(self, gdn_index: int) -> np.ndarray:
        """Recurrent state [n_v][hd][hd] of the gdn_index-th Gated-DeltaNet layer."""
        c = self.cfg
        out = np.empty((c.ssm_n_v_heads, c.ssm_head_dim, c.ssm_head_dim), np.float32)
        _check(self.lib.hh_model_download_state(self.h, gdn_index, out.ctypes.data, out.size))
        return out

    def set_hadamard_signs(self, width: int, signs: np.ndarray) -> None:
        """Sign vector of one Hadamard fold width (qwen35.rs:561-586, :843-845)."""
        s = np.ascontiguousarray(signs, dtype=np.float32)
        if s.size != width:
            raise ValueError("signs must hold `width` values")
        _check(self.lib.hh_model_set_hadamard_signs(self.h, width, s.ctypes.data))

    def upload(self, name: str, ggml_type: int, ne0: int, ne1: int, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data)
        _check(self.lib.hh_model_upload_tensor(self.h, name.encode(), ggml_type, ne0, ne1,
                                               data.ctypes.data, data.nbytes))

    def download(self, name: str, nbytes: int) -> np.ndarray:
        buf = np.empty(nbytes, dtype=np.uint8)
        _check(self.lib.hh_model_download_tensor(self.h, name.encode(), buf.ctypes.data, nbytes))
        return buf

    def set_cancel(self, flag: bool) -> None:
        _check(self.lib.hh_model_set_cancel(self.h, int(flag)))

    def forward(self, token: int, pos: int, want_logits: bool = True):
        logits = np.empty(self.cfg.vocab, dtype=np.float32) if want_logits else None
        am = C.c_uint32()
        _check(self.lib.hh_model_forward(self.h, token, pos, logits.ctypes.data if want_logits else None,
                                         C.byref(am)))
        return logits, am.value

    def generate(self, prompt: Sequence[int], n_gen: int, start_pos: int = 0, repeat_pen: float = 1.0,
                 want_logits: bool = False):
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.uint32))
        toks = np.zeros(max(n_gen, 1), dtype=np.uint32)
        logits = np.empty(self.cfg.vocab, dtype=np.float32) if want_logits else None
        _check(self.lib.hh_model_generate(self.h, p.ctypes.data, len(p), start_pos, n_gen, repeat_pen,
                                          toks.ctypes.data, logits.ctypes.data if want_logits else None))
        return toks[:n_gen], logits

    STAGES = ("embed", "in_proj", "mix", "out_proj", "gate_up", "down", "head")

    def time_stages(self, layer: int = 0, iters: int = 20) -> dict:
        out = np.zeros(7, dtype=np.float64)
        _check(self.lib.hh_model_time_stages(self.h, layer, iters, out.ctypes.data, 7))
        return dict(zip(self.STAGES, out.tolist()))

    def prefill(self, tokens: Sequence[int], start_pos: int = 0) -> None:
        """Batched prefill: K/V (and GDN state) for tokens at start_pos.., no logits."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        _check(self.lib.hh_model_prefill(self.h, t.ctypes.data, len(t), start_pos))

    def last_prefill_ms(self) -> float:
        v = C.c_double()
        _check(self.lib.hh_model_last_prefill_ms(self.h, C.byref(v)))
        return v.value

    def last_decode_ms(self) -> float:
        v = C.c_double()
        _check(self.lib.hh_model_last_decode_ms(self.h, C.byref(v)))
        return v.value
