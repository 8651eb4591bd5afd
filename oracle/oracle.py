"""ctypes binding of the CPU oracle (oracle/hearth_oracle.c).

TEST INFRASTRUCTURE ONLY — loaded by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product (hearth_amd/).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
_LIB: Optional[C.CDLL] = None


class HoConfig(C.Structure):
    _fields_ = [
        ("arch", C.c_int), ("d_model", C.c_int), ("n_layers", C.c_int), ("n_heads", C.c_int),
        ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("d_ffn", C.c_int), ("vocab", C.c_int),
        ("eps", C.c_float), ("rope_theta", C.c_float), ("rope_dim", C.c_int), ("max_seq", C.c_int),
        ("wtype", C.c_int), ("head_type", C.c_int), ("qk_norm", C.c_int),
        ("full_attn_interval", C.c_int), ("ssm_n_k_heads", C.c_int), ("ssm_n_v_heads", C.c_int),
        ("ssm_head_dim", C.c_int), ("ssm_conv_kernel", C.c_int), ("attn_out_gate", C.c_int),
        ("kv_type", C.c_int), ("had_block", C.c_int), ("had_flags", C.c_int),
    ]


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def load() -> C.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        build()
    lib = C.CDLL(LIB_PATH)
    u8p, f32p, u32p = C.c_void_p, C.c_void_p, C.c_void_p
    sig = {
        "ho_f32_to_f16": (C.c_uint16, [C.c_float]),
        "ho_f16_to_f32": (C.c_float, [C.c_uint16]),
        "ho_row_bytes": (C.c_size_t, [C.c_int, C.c_int64]),
        "ho_quantize_q8_0": (None, [f32p, C.c_int64, u8p]),
        "ho_dequantize": (C.c_int, [C.c_int, u8p, C.c_int64, f32p]),
        "ho_dot_q2_0_q8_0": (C.c_float, [u8p, u8p, C.c_int64]),
        "ho_dot_q1_0_q8_0": (C.c_float, [u8p, u8p, C.c_int64]),
        "ho_dot_q8_0_q8_0": (C.c_float, [u8p, u8p, C.c_int64]),
        "ho_dot_ptq1_0_q8_0": (C.c_float, [u8p, u8p, C.c_int64]),
        "ho_quantize_ptq1_0": (None, [f32p, C.c_int64, u8p]),
        "ho_ptq1_0_pack_codes": (None, [C.c_void_p, C.c_uint16, u8p]),
        "ho_dot_q2_0_q8_0_avx2": (C.c_float, [u8p, u8p, C.c_int64]),
        "ho_dot_q1_0_q8_0_avx2": (C.c_float, [u8p, u8p, C.c_int64]),
        "ho_have_avx2": (C.c_int, []),
        "ho_gemv": (C.c_int, [C.c_int, u8p, C.c_int64, C.c_int64, u8p, f32p, C.c_int, C.c_int]),
        "ho_rms_norm": (None, [f32p, f32p, C.c_float, C.c_int64, f32p]),
        "ho_rope_table": (None, [C.c_int, C.c_int, C.c_float, f32p]),
        "ho_rope_apply": (None, [f32p, C.c_int, C.c_int, f32p, C.c_int]),
        "ho_silu": (None, [f32p, C.c_int64]),
        "ho_softmax": (None, [f32p, C.c_int64]),
        "ho_attention": (None, [f32p, f32p, f32p, C.c_int, C.c_int, f32p, f32p]),
        "ho_attn_chunk": (C.c_int, [C.c_int, C.c_int, C.c_int]),
        "ho_attention_dev": (None, [f32p, f32p, f32p, C.c_int, C.c_int, C.c_int, f32p]),
        "ho_sample_greedy_dense": (C.c_uint32, [f32p, C.c_int64, u32p, C.c_int64, C.c_float]),
        "ho_argmax_first": (C.c_uint32, [f32p, C.c_int64]),
        "ho_name_key": (C.c_uint64, [C.c_uint64, C.c_char_p]),
        "ho_synth_int": (C.c_int32, [C.c_uint64, C.c_uint64]),
        "ho_synth_scale": (C.c_float, [C.c_float]),
        "ho_synth_tensor": (None, [C.c_int, C.c_uint64, C.c_char_p, C.c_int64, C.c_int64, C.c_float, C.c_float,
                                   C.c_void_p, C.c_int]),
        "ho_synth_token": (C.c_uint32, [C.c_uint64, C.c_int64, C.c_uint32]),
        "ho_model_new": (C.c_void_p, [C.POINTER(HoConfig)]),
        "ho_model_free": (None, [C.c_void_p]),
        "ho_model_tensor": (C.c_void_p, [C.c_void_p, C.c_char_p, C.POINTER(C.c_size_t), C.POINTER(C.c_int),
                                         C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
        "ho_model_tensor_count": (C.c_int, [C.c_void_p]),
        "ho_model_tensor_name": (C.c_char_p, [C.c_void_p, C.c_int]),
        "ho_model_synth": (None, [C.c_void_p, C.c_uint64, C.c_int]),
        "ho_model_reset": (None, [C.c_void_p]),
        "ho_model_kv_prefill_synth": (C.c_int, [C.c_void_p, C.c_uint64, C.c_int]),
        "ho_model_set_threads": (None, [C.c_void_p, C.c_int, C.c_int]),
        "ho_model_set_order": (None, [C.c_void_p, C.c_int]),
        "ho_exp": (C.c_float, [C.c_float]),
        "ho_log": (C.c_float, [C.c_float]),
        "ho_forward": (C.c_int, [C.c_void_p, C.c_uint32, C.c_int, f32p]),
        "ho_generate": (C.c_int, [C.c_void_p, u32p, C.c_int, C.c_int, C.c_int, C.c_float, u32p, f32p]),
        "ho_model_hidden": (C.c_void_p, [C.c_void_p]),
        "ho_model_buffer": (C.c_void_p, [C.c_void_p, C.c_int]),
        "ho_model_q8_trace": (None, [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t]),
        "ho_model_q8_trace_stats": (C.c_size_t, [C.c_void_p, C.c_void_p]),
        "ho_wht": (None, [f32p, C.c_int64]),
        "ho_hadamard_rotate": (None, [f32p, C.c_int64, C.c_void_p, C.c_int]),
        "ho_hadamard_unrotate": (None, [f32p, C.c_int64, C.c_void_p, C.c_int]),
        "ho_model_set_signs": (C.c_int, [C.c_void_p, C.c_int, f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


# ---- numpy-friendly wrappers ----
def f32_to_f16(x: float) -> int:
    return load().ho_f32_to_f16(x)


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros((x.size + 31) // 32 * 34, dtype=np.uint8)
    load().ho_quantize_q8_0(_p(x), x.size, _p(out))
    return out


def dequantize(t: int, w: np.ndarray, n: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.zeros(n, dtype=np.float32)
    rc = load().ho_dequantize(t, _p(w), n, _p(out))
    assert rc == 0
    return out


def quantize_ptq1_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 128 * 28, dtype=np.uint8)
    load().ho_quantize_ptq1_0(_p(x), x.size, _p(out))
    return out


def ptq1_0_pack_codes(codes: np.ndarray, f16_scale: int) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.int32)
    assert c.size == 128
    out = np.zeros(28, dtype=np.uint8)
    load().ho_ptq1_0_pack_codes(_p(c), f16_scale, _p(out))
    return out


def dot(t: int, w: np.ndarray, a: np.ndarray, n: int, avx2: bool = False) -> float:
    lib = load()
    fn = {42: "q2_0", 142: "q2_0", 41: "q1_0", 43: "q1_0", 8: "q8_0", 143: "ptq1_0"}[t]
    name = f"ho_dot_{fn}_q8_0" + ("_avx2" if avx2 else "")
    return getattr(lib, name)(_p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(a)), n)


def gemv(t: int, w: np.ndarray, n_rows: int, n_cols: int, a: np.ndarray, threads: int = 1,
         arm: int = 0) -> np.ndarray:
    y = np.zeros(n_rows, dtype=np.float32)
    rc = load().ho_gemv(t, _p(np.ascontiguousarray(w)), n_rows, n_cols, _p(np.ascontiguousarray(a)), _p(y),
                        threads, arm)
    assert rc == 0
    return y


def synth_tensor(t: int, seed: int, name: str, rows: int, cols: int, std: float, mean: float,
                 threads: int = 4) -> np.ndarray:
    lib = load()
    nb = lib.ho_row_bytes(t, cols) * rows
    out = np.zeros(nb, dtype=np.uint8)
    lib.ho_synth_tensor(t, seed, name.encode(), rows, cols, std, mean, _p(out), threads)
    return out


def wht(x: np.ndarray) -> np.ndarray:
    y = np.array(x, dtype=np.float32)
    load().ho_wht(_p(y), y.size)
    return y


def hadamard_rotate(x: np.ndarray, signs, block: int, inverse: bool = False) -> np.ndarray:
    y = np.array(x, dtype=np.float32)
    s = None if signs is None else np.ascontiguousarray(signs, dtype=np.float32)
    fn = load().ho_hadamard_unrotate if inverse else load().ho_hadamard_rotate
    fn(_p(y), y.size, None if s is None else _p(s), block)
    return y


def synth_token(seed: int, i: int, vocab: int) -> int:
    return load().ho_synth_token(seed, i, vocab)


class OracleModel:
    REFERENCE, DEVICE = 0, 1

    def __init__(self, cfg, seed: Optional[int] = None, threads: int = 4, arm: int = 0, order: int = 0):
        self.lib = load()
        self.cfg = cfg
        self._c = HoConfig(*[getattr(cfg, f[0]) for f in HoConfig._fields_])
        self.h = self.lib.ho_model_new(C.byref(self._c))
        self.lib.ho_model_set_threads(self.h, threads, arm)
        self.lib.ho_model_set_order(self.h, order)
        if seed is not None:
            self.lib.ho_model_synth(self.h, seed, threads)

    def close(self):
        if self.h:
            self.lib.ho_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_signs(self, width: int, signs: np.ndarray) -> None:
        s = np.ascontiguousarray(signs, dtype=np.float32)
        assert s.size == width
        assert self.lib.ho_model_set_signs(self.h, width, _p(s)) == 0
        self._signs = getattr(self, "_signs", []) + [s]

    def q8_trace(self, mode: int, buf: Optional[np.ndarray] = None) -> None:
        """Diagnostics: mode 1 records every matmul input's Q8_0 bytes into buf,
        mode 2 replays them in place of the model's own quantization, 0 = off."""
        self._trace = buf
        self.lib.ho_model_q8_trace(self.h, mode, None if buf is None else buf.ctypes.data,
                                   0 if buf is None else buf.nbytes)

    def q8_trace_stats(self):
        """(bytes used, replayed bytes that differed, matmul inputs with a differing byte)"""
        st = np.zeros(2, dtype=np.int64)
        n = self.lib.ho_model_q8_trace_stats(self.h, st.ctypes.data)
        return int(n), int(st[0]), int(st[1])

    def set_order(self, order: int) -> None:
        self.lib.ho_model_set_order(self.h, order)

    def set_threads(self, threads: int, arm: int) -> None:
        self.lib.ho_model_set_threads(self.h, threads, arm)

    def tensor(self, name: str) -> np.ndarray:
        nb = C.c_size_t()
        p = self.lib.ho_model_tensor(self.h, name.encode(), C.byref(nb), None, None, None)
        if not p:
            raise KeyError(name)
        return np.ctypeslib.as_array((C.c_uint8 * nb.value).from_address(p))

    def tensor_names(self):
        return [self.lib.ho_model_tensor_name(self.h, i).decode() for i in range(self.lib.ho_model_tensor_count(self.h))]

    def reset(self):
        self.lib.ho_model_reset(self.h)

    def prefill_kv_synthetic(self, seed: int, n_pos: int) -> None:
        assert self.lib.ho_model_kv_prefill_synth(self.h, seed, n_pos) == 0

    def forward(self, token: int, pos: int) -> np.ndarray:
        logits = np.zeros(self.cfg.vocab, dtype=np.float32)
        rc = self.lib.ho_forward(self.h, token, pos, _p(logits))
        assert rc == 0, rc
        return logits

    def generate(self, prompt: Sequence[int], n_gen: int, start_pos: int = 0, repeat_pen: float = 1.0,
                 want_logits: bool = False):
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.uint32))
        toks = np.zeros(max(n_gen, 1), dtype=np.uint32)
        logits = np.zeros(self.cfg.vocab, dtype=np.float32) if want_logits else None
        rc = self.lib.ho_generate(self.h, _p(p), len(p), start_pos, n_gen, repeat_pen, _p(toks),
                                  _p(logits) if want_logits else None)
        assert rc == 0, rc
        return toks[:n_gen], logits
