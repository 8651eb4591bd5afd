"""CPU pins of the oracle's block formats and dot kernels.

Each check is independent of the oracle's own formula: numpy float16 (IEEE
RNE) for the f16 conversion, the reference tests' known answers, a numpy
restatement for Q8_0, brute-force float64 dots from dequantized operands.
"""
import numpy as np
import pytest

from tests.fixtures import (exact_dot, np_dequant, np_quantize_q8_0, ref_act, ref_q1_weights,
                            ref_q2_weights)


def test_f16_matches_numpy_rne(oracle):
    lib = oracle.load()
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 6, 200000),
        np.array([0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6e-8, 5.96e-8, 2.98e-8, 3e-8,
                  6.1e-5, 6.09e-5, np.inf, -np.inf], dtype=np.float32),
        # exact ties between f16 neighbours (round-half-even cases)
        (np.arange(1, 2000, dtype=np.float32) * np.float32(2.0 ** -11) + np.float32(1.0)),
    ]).astype(np.float32)
    with np.errstate(over='ignore'):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([lib.ho_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)
    # and back: exact widening
    h = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    finite = h[(h & 0x7C00) != 0x7C00]
    back = np.array([lib.ho_f16_to_f32(int(x)) for x in finite[::7]], dtype=np.float32)
    assert np.array_equal(back, finite[::7].view(np.float16).astype(np.float32))


def test_q8_0_known_answers(oracle):
    # all-zero block: scale 1.0 (0x3C00), q = 0 (q8_0.rs:35)
    q = oracle.quantize_q8_0(np.zeros(32, np.float32))
    assert q[0] == 0x00 and q[1] == 0x3C and not q[2:].any()
    # a block whose max is 127: scale exactly 1.0 and q = x
    x = np.arange(-15, 17, dtype=np.float32)
    x[5] = 127.0
    q = oracle.quantize_q8_0(x)
    assert q[0] == 0x00 and q[1] == 0x3C
    assert np.array_equal(q[2:].view(np.int8), x.astype(np.int8))
    # half-way values round away from zero: 0.5*s -> 1, -0.5*s -> -1
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2] = 127.0, 0.5, -0.5
    q = oracle.quantize_q8_0(x).view(np.int8)
    assert (q[2], q[3], q[4]) == (127, 1, -1)
    # tail handling: n not a multiple of 32 zero-pads (q8_0.rs:41-47)
    q = oracle.quantize_q8_0(np.ones(40, np.float32))
    assert len(q) == 68 and not q[34 + 2 + 8:].any()


def test_q8_0_matches_numpy_restatement(oracle):
    rng = np.random.default_rng(1)
    for scale in (1e-3, 1.0, 37.0):
        x = (rng.standard_normal(4096) * scale).astype(np.float32)
        assert np.array_equal(oracle.quantize_q8_0(x), np_quantize_q8_0(x))


def test_q8_0_roundtrip_and_dot(oracle):
    # q8_0.rs:177-212: round-trip error < 1.0 and the dot within 2%
    src = (np.arange(64, dtype=np.float32) - 32.0) * 0.5
    q = oracle.quantize_q8_0(src)
    deq = oracle.dequantize(8, q, 64)
    assert np.abs(src - deq).max() < 1.0


def test_q2_0_dequant_known_answers(oracle):
    # q2_0.rs:738-766 / pq2_0.rs:79-93: 0b00100100 at scale 2.0 -> [-2, 0, +2, -2]
    data = np.zeros(68, np.uint8)
    data[0:2] = np.frombuffer(np.float16(2.0).tobytes(), np.uint8)
    data[2] = 0b00100100
    for t in (42, 142):
        out = oracle.dequantize(t, data, 256)
        assert list(out[:4]) == [-2.0, 0.0, 2.0, -2.0]
    # q2_0.rs:913-934: 0xAA -> all +1
    w = np.zeros(34, np.uint8)
    w[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    w[2:] = 0xAA
    assert np.all(oracle.dequantize(42, w, 128) == 1.0)


def test_q1_0_dequant_known_answers(oracle):
    # q1_0g128.rs:1459-1502: all bits 1 -> +scale, all 0 -> -scale
    w = np.zeros(18, np.uint8)
    w[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    w[2:] = 0xFF
    assert np.all(oracle.dequantize(41, w, 128) == 0.5)
    w[0:2] = np.frombuffer(np.float16(1.5).tobytes(), np.uint8)
    w[2:] = 0x00
    assert np.all(oracle.dequantize(43, w, 128) == -1.5)
    # bit j of byte i is element 8i+j (LSB first)
    w[2:] = 0
    w[3] = 0b00000100   # element 8 + 2
    out = oracle.dequantize(41, w, 128)
    assert out[10] == 1.5 and (out[np.arange(128) != 10] == -1.5).all()


@pytest.mark.parametrize("t", [8, 41, 42])
def test_dequant_matches_numpy(oracle, t):
    rng = np.random.default_rng(t)
    n = 1024
    nb = {8: n // 32 * 34, 41: n // 128 * 18, 42: n // 128 * 34}[t]
    w = rng.integers(0, 256, nb, dtype=np.uint8)
    bs = {8: 34, 41: 18, 42: 34}[t]
    for b in range(nb // bs):   # finite scales
        w[b * bs:b * bs + 2] = np.frombuffer(np.float16(rng.uniform(-2, 2)).tobytes(), np.uint8)
    assert np.array_equal(oracle.dequantize(t, w, n), np_dequant(t, w, n))


@pytest.mark.parametrize("n", [128, 256, 2048, 6144])
def test_dots_on_reference_generators(oracle, n):
    """q2_0.rs:939-986 / q1_0g128.rs:1504-1551 fixtures: the scalar dots equal the
    exact value of the dequantized operands to fp32 accumulation accuracy, the
    AVX2 arms agree with the scalar ones, and the fixture is not degenerate."""
    w2, w1 = ref_q2_weights(n), ref_q1_weights(n)
    for salt in (53, 97):
        a = ref_act(n, salt)
        for t, w in ((42, w2), (41, w1)):
            s = oracle.dot(t, w, a, n)
            ex = exact_dot(t, w, a, n)
            assert abs(s) > 1e-6
            assert abs(s - ex) <= 1e-5 * max(1.0, abs(ex)) + 1e-3
            has_m128 = bool((a.reshape(-1, 34)[:, 2:] == 0x80).any())
            if oracle.load().ho_have_avx2() and not (t == 41 and has_m128):
                v = oracle.dot(t, w, a, n, avx2=True)
                assert abs(v - s) <= 1e-5 * max(1.0, abs(s))


def test_q1_avx2_arm_diverges_only_on_minus_128(oracle):
    """The shipped Q1 AVX2 arm negates activations with (a ^ m) - m
    (q1_0g128.rs:300-301), which wraps for a = -128; the scalar kernel and the
    GPU kernel compute the exact sum.  Q8_0 quantization never emits -128
    (|x/scale| <= 127), so the arms agree on every quantized activation."""
    if not oracle.load().ho_have_avx2():
        pytest.skip("host lacks AVX2")
    n = 6144
    w = ref_q1_weights(n)
    a = ref_act(n, 53)
    assert oracle.dot(41, w, a, n) != oracle.dot(41, w, a, n, avx2=True)
    a2 = a.copy().reshape(-1, 34)
    a2[:, 2:][a2[:, 2:] == 0x80] = 0x81
    a2 = a2.reshape(-1)
    s, v = oracle.dot(41, w, a2, n), oracle.dot(41, w, a2, n, avx2=True)
    assert abs(s - v) <= 1e-5 * max(1.0, abs(s))
    rng = np.random.default_rng(11)
    q = oracle.quantize_q8_0((rng.standard_normal(1 << 16) * 50).astype(np.float32))
    assert not (q.reshape(-1, 34)[:, 2:] == 0x80).any()


def test_q8_0_dot_exact(oracle):
    rng = np.random.default_rng(3)
    n = 4096
    x = rng.standard_normal(n).astype(np.float32)
    y = rng.standard_normal(n).astype(np.float32)
    w, a = oracle.quantize_q8_0(x), oracle.quantize_q8_0(y)
    s = oracle.dot(8, w, a, n)
    assert abs(s - exact_dot(8, w, a, n)) < 1e-4 * n ** 0.5


def test_dot_brute_force_tiny(oracle):
    """Exhaustive small cases: every code value against every activation sign."""
    rng = np.random.default_rng(4)
    for _ in range(50):
        w = rng.integers(0, 256, 34, dtype=np.uint8)
        w[0:2] = np.frombuffer(np.float16(rng.uniform(0.1, 2)).tobytes(), np.uint8)
        a = oracle.quantize_q8_0(rng.standard_normal(128).astype(np.float32))
        assert abs(oracle.dot(42, w, a, 128) - exact_dot(42, w, a, 128)) < 1e-4
        w1 = w[:18].copy()
        assert abs(oracle.dot(41, w1, a, 128) - exact_dot(41, w1, a, 128)) < 1e-4


def test_gemv_partitioning_matches_rowwise(oracle):
    """pool.rs:321-347: contiguous ceil(N/T) chunks give the same rows as a serial loop."""
    rng = np.random.default_rng(5)
    n_rows, n_cols = 37, 512
    w = oracle.synth_tensor(42, 9, "w", n_rows, n_cols, 0.02, 0.0)
    a = oracle.quantize_q8_0(rng.standard_normal(n_cols).astype(np.float32))
    y1 = oracle.gemv(42, w, n_rows, n_cols, a, threads=1)
    y4 = oracle.gemv(42, w, n_rows, n_cols, a, threads=4)
    assert np.array_equal(y1, y4)
    rb = n_cols // 128 * 34
    for r in range(n_rows):
        assert y1[r] == oracle.dot(42, w[r * rb:(r + 1) * rb], a, n_cols)
