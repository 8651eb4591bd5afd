"""Property tests of the CPU oracle (hypothesis), pinning it from directions
the known-answer tests leave open:

* Q8_0 (q8_0.rs:20-51): every code in [-127, 127], the stored scale is the f16
  of max|x| / 127, each value within half a step of its dequantized form, and
  quantizing the dequantized block returns the same bytes (unless the scale
  underflowed f16 to zero).
* Q2_0 / Q1_0 / PQ2_0 / PTQ1_0 dequantization of arbitrary bytes equals an
  independent numpy decode of the block layout (q2_0.rs:66-84, pq2_0.rs:32-50,
  q1_0g128.rs:75-98, ptq1_0.rs:6-13).
* The Q8_0-activation dot of every format equals the float64 dot of the two
  dequantized operands (to f32 rounding), and is linear in the activation
  block scales: doubling every activation scale doubles the dot exactly.
"""
import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

GGML_Q8_0, GGML_Q1_0, GGML_Q2_0, GGML_Q1_0_G128, GGML_PQ2_0, GGML_PTQ1_0 = 8, 41, 42, 43, 142, 143
BLOCK = {GGML_Q1_0: (128, 18), GGML_Q1_0_G128: (128, 18), GGML_Q2_0: (128, 34), GGML_PQ2_0: (128, 34),
         GGML_PTQ1_0: (128, 28)}
SETTINGS = settings(max_examples=40, deadline=None, derandomize=True)   # deterministic suite


def _f16(b0, b1):
    return float(np.frombuffer(bytes([b0, b1]), np.float16)[0])


def _numpy_decode(t, w):
    """Independent decode of the block layouts (not the oracle's code)."""
    el, bb = BLOCK[t]
    out = []
    for blk in w.reshape(-1, bb):
        if t == GGML_PTQ1_0:
            d = _f16(blk[26], blk[27])
            vals = np.zeros(128)
            for n in range(5):              # qs: 5 trits per byte, the n-th base-3 digit
                for m in range(24):
                    q = ((int(blk[m]) * 3 ** n) % 256) * 3 >> 8
                    e = 16 * n + m if m < 16 else 80 + 8 * n + (m - 16)
                    vals[e] = q - 1
            for n in range(4):              # qh: 4 trits per byte
                for hbyte in range(2):
                    q = ((int(blk[24 + hbyte]) * 3 ** n) % 256) * 3 >> 8
                    vals[120 + 2 * n + hbyte] = q - 1
            out.append(vals * d)
            continue
        d = _f16(blk[0], blk[1])
        qs = blk[2:]
        if t in (GGML_Q2_0, GGML_PQ2_0):   # both map code c to c - 1 (pq2_0.rs:3, :14-27)
            codes = np.array([(qs[i // 4] >> (2 * (i % 4))) & 3 for i in range(128)], np.float64)
            out.append((codes - 1.0) * d)
        else:
            bits = np.array([(qs[i // 8] >> (i % 8)) & 1 for i in range(128)], np.float64)
            out.append((2.0 * bits - 1.0) * d)
    return np.concatenate(out)


def _finite_scale_blocks(t, raw, scales):
    """Arbitrary code bytes with finite, moderate f16 block scales."""
    el, bb = BLOCK[t]
    w = np.frombuffer(raw, np.uint8).copy()
    off = 26 if t == GGML_PTQ1_0 else 0
    for b, s in enumerate(scales):
        h = np.float16(s).view(np.uint16)
        w[b * bb + off], w[b * bb + off + 1] = int(h) & 0xFF, int(h) >> 8
    return w


floats = st.floats(min_value=-1e4, max_value=1e4, allow_nan=False, allow_infinity=False, width=32)


@SETTINGS
@given(st.integers(min_value=1, max_value=8).flatmap(lambda nb: st.lists(floats, min_size=32 * nb, max_size=32 * nb)))
def test_q8_0_bounds_and_idempotence(oracle, vals):
    x = np.array(vals, np.float32)
    q = oracle.quantize_q8_0(x)
    assert q.size == x.size // 32 * 34
    blocks = q.reshape(-1, 34)
    codes = blocks[:, 2:].view(np.int8).astype(np.int32)
    assert codes.min() >= -127 and codes.max() <= 127
    deq = oracle.dequantize(GGML_Q8_0, q, x.size)
    for b in range(x.size // 32):
        xb = x[32 * b:32 * b + 32].astype(np.float64)
        amax = np.abs(xb).max()
        d = _f16(blocks[b, 0], blocks[b, 1])
        want = np.float32(np.float32(amax) / np.float32(127.0)) if amax > 0 else np.float32(1.0)
        assert d == float(np.float16(want))           # the f16 of max|x| / 127 (1 for a zero block)
        step = float(want)
        assert np.all(np.abs(deq[32 * b:32 * b + 32] - xb) <= 0.5 * step * 1.0001 + abs(d - step) * 127 + 1e-30)
    # idempotent unless a nonzero block's scale underflowed f16 to 0 (max|x| < ~1.1e-5 * 2^-14):
    # its dequantized block is all zero and re-quantizes with scale 1 (q8_0.rs:35)
    d_all = blocks[:, :2].copy().view(np.float16).astype(np.float32).ravel()
    amax_all = np.abs(x.reshape(-1, 32)).max(axis=1)
    if not np.any((d_all == 0) & (amax_all > 0)):
        assert np.array_equal(oracle.quantize_q8_0(deq), q)


@SETTINGS
@given(st.sampled_from([GGML_Q1_0, GGML_Q1_0_G128, GGML_Q2_0, GGML_PQ2_0, GGML_PTQ1_0]),
       st.integers(min_value=1, max_value=4).flatmap(
           lambda nb: st.tuples(st.just(nb), st.binary(min_size=nb * 34, max_size=nb * 34),
                                st.lists(st.floats(min_value=1e-3, max_value=4.0), min_size=nb, max_size=nb))))
def test_dequantize_matches_independent_decode(oracle, t, args):
    nb, raw, scales = args
    el, bb = BLOCK[t]
    w = _finite_scale_blocks(t, raw[:nb * bb], scales)
    got = oracle.dequantize(t, w, nb * 128).astype(np.float64)
    assert np.array_equal(got, _numpy_decode(t, w))


@SETTINGS
@given(st.sampled_from([GGML_Q1_0, GGML_Q2_0, GGML_PQ2_0, GGML_PTQ1_0]),
       st.integers(min_value=1, max_value=3).flatmap(
           lambda nb: st.tuples(st.just(nb), st.binary(min_size=nb * 34, max_size=nb * 34),
                                st.lists(st.floats(min_value=1e-2, max_value=2.0), min_size=nb, max_size=nb),
                                st.lists(floats, min_size=nb * 128, max_size=nb * 128))))
def test_dot_against_float64_and_scale_linearity(oracle, t, args):
    nb, raw, scales, avals = args
    el, bb = BLOCK[t]
    n = nb * 128
    w = _finite_scale_blocks(t, raw[:nb * bb], scales)
    a = oracle.quantize_q8_0(np.array(avals, np.float32))
    got = oracle.dot(t, w, a, n)
    want = float(np.dot(oracle.dequantize(t, w, n).astype(np.float64),
                        oracle.dequantize(GGML_Q8_0, a, n).astype(np.float64)))
    mag = float(np.dot(np.abs(oracle.dequantize(t, w, n).astype(np.float64)),
                       np.abs(oracle.dequantize(GGML_Q8_0, a, n).astype(np.float64))))
    assert abs(got - want) <= 2e-6 * max(mag, 1e-30)
    # doubling every activation block scale (exact in f16 unless it overflows) doubles the dot
    a2 = a.copy().reshape(-1, 34)
    s = a2[:, :2].copy().view(np.float16).astype(np.float32) * 2
    if np.all(np.isfinite(s.astype(np.float16))) and np.all(np.abs(s) < 6e4):
        a2[:, :2] = s.astype(np.float16).view(np.uint8).reshape(-1, 2)
        assert oracle.dot(t, w, a2.reshape(-1), n) == 2.0 * got
