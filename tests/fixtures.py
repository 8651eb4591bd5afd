"""Deterministic byte generators restated from the reference's own tests.

q2_0.rs:939-986 and q1_0g128.rs:1504-1551 (paired-vs-single fixtures):
weights w[b*BB + 2 + j] = ((b*NB + j) * 37) ^ 0xAB, scale f16(((b % 7) + 0.5) * 0.25);
activations act[b*34 + 2 + j] = (b * salt * 2654435761) as u8, scale f16(((b % 5) + 0.5) * 0.125).
"""
import numpy as np


def f16_bytes(x: float) -> bytes:
    return np.float16(x).tobytes()


def ref_q2_weights(n: int) -> np.ndarray:
    nb = n // 128
    w = np.zeros(nb * 34, dtype=np.uint8)
    for b in range(nb):
        w[b * 34:b * 34 + 2] = np.frombuffer(f16_bytes(((b % 7) + 0.5) * 0.25), dtype=np.uint8)
        for j in range(32):
            w[b * 34 + 2 + j] = (((b * 32 + j) * 37) ^ 0xAB) & 0xFF
    return w


def ref_q1_weights(n: int) -> np.ndarray:
    nb = n // 128
    w = np.zeros(nb * 18, dtype=np.uint8)
    for b in range(nb):
        w[b * 18:b * 18 + 2] = np.frombuffer(f16_bytes(((b % 7) + 0.5) * 0.25), dtype=np.uint8)
        for j in range(16):
            w[b * 18 + 2 + j] = (((b * 16 + j) * 37) ^ 0xAB) & 0xFF
    return w


def ref_act(n: int, salt: int) -> np.ndarray:
    nb = n // 32
    a = np.zeros(nb * 34, dtype=np.uint8)
    for b in range(nb):
        a[b * 34:b * 34 + 2] = np.frombuffer(f16_bytes(((b % 5) + 0.5) * 0.125), dtype=np.uint8)
        a[b * 34 + 2:b * 34 + 34] = ((b * salt * 2654435761) & 0xFFFFFFFF) & 0xFF
    return a


def np_dequant_q8(a: np.ndarray, n: int) -> np.ndarray:
    blk = a.reshape(-1, 34)[: n // 32]
    d = blk[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1, 1)
    return (d * blk[:, 2:].view(np.int8).astype(np.float32)).reshape(-1)


def np_dequant(t: int, w: np.ndarray, n: int) -> np.ndarray:
    """Independent numpy dequantizer (q8_0.rs:4-18, q2_0.rs:66-84, q1_0g128.rs:75-98)."""
    if t == 8:
        return np_dequant_q8(w, n)
    if t in (42, 142):
        blk = w.reshape(-1, 34)[: n // 128]
        d = blk[:, :2].copy().view(np.float16).astype(np.float32)
        codes = np.stack([(blk[:, 2:] >> (2 * k)) & 3 for k in range(4)], axis=-1).reshape(-1, 128)
        return ((codes.astype(np.float32) - 1.0) * d).reshape(-1)
    if t in (41, 43):
        blk = w.reshape(-1, 18)[: n // 128]
        d = blk[:, :2].copy().view(np.float16).astype(np.float32)
        bits = np.stack([(blk[:, 2:] >> k) & 1 for k in range(8)], axis=-1).reshape(-1, 128)
        return ((bits.astype(np.float32) * 2.0 - 1.0) * d).reshape(-1)
    raise ValueError(t)


def exact_dot(t: int, w: np.ndarray, a: np.ndarray, n: int) -> float:
    """Brute-force value of the dot in float64 from the dequantized operands."""
    return float(np.dot(np_dequant(t, w, n).astype(np.float64), np_dequant_q8(a, n).astype(np.float64)))


def np_quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """Independent numpy statement of q8_0.rs:20-51 (round half away from zero)."""
    x = np.asarray(x, dtype=np.float32)
    n = x.size
    nb = (n + 31) // 32
    xp = np.zeros(nb * 32, dtype=np.float32)
    xp[:n] = x
    xb = xp.reshape(nb, 32)
    amax = np.abs(xb).max(axis=1)
    scale = np.where(amax == 0, np.float32(1.0), (amax / np.float32(127.0)).astype(np.float32)).astype(np.float32)
    v = xb / scale[:, None]
    v64 = v.astype(np.float64)
    r = np.sign(v64) * np.floor(np.abs(v64) + 0.5)
    q = np.clip(r, -128, 127).astype(np.int8)
    out = np.zeros((nb, 34), dtype=np.uint8)
    out[:, :2] = scale.astype(np.float16).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)
