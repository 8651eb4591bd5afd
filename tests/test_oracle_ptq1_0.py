"""PTQ1_0 (GGML type 143) in the CPU oracle, pinned without running the reference.

* Closed form: byte ceil(256*Q/243) must decode, slot by slot, to the base-3
  digits of Q (ptq1_0.rs:6-13), for every Q the format can hold.
* Known answers from the reference's own tests (ptq1_0.rs:652-756).
* The q8 dot against an independent float64 sum over dequantized operands, and
  exactly against the integer dot when the activation scales are 1.
* Idempotence: quantizing dequantized weights returns the same bytes.
* The synthesized PTQ1_0 weights equal the Q2_0 generator's weights.
"""
import numpy as np
import pytest

GGML_Q2_0, GGML_PTQ1_0 = 42, 143


def _digits(q, k):
    return [(q // 3 ** (k - 1 - i)) % 3 for i in range(k)]


def test_trit_decode_closed_form(oracle):
    f16_one = oracle.f32_to_f16(1.0)
    for q in range(243):
        b = (256 * q + 242) // 243
        blk = np.zeros(28, np.uint8)
        blk[:24] = b
        blk[26], blk[27] = f16_one & 0xFF, f16_one >> 8
        w = oracle.dequantize(GGML_PTQ1_0, blk, 128)
        d = _digits(q, 5)
        for n in range(5):
            # stage A: element 16n + m (m < 16); stage B: element 80 + 8n + (m - 16)
            assert all(w[16 * n + m] == d[n] - 1 for m in range(16)), (q, n)
            assert all(w[80 + 8 * n + m] == d[n] - 1 for m in range(8)), (q, n)
    for q in range(81):   # qh: four trits and a trailing zero trit
        b = (256 * 3 * q + 242) // 243
        blk = np.zeros(28, np.uint8)
        blk[24] = blk[25] = b
        blk[26], blk[27] = f16_one & 0xFF, f16_one >> 8
        w = oracle.dequantize(GGML_PTQ1_0, blk, 128)
        d = _digits(q, 4)
        for n in range(4):
            assert w[120 + 2 * n] == d[n] - 1 and w[121 + 2 * n] == d[n] - 1, (q, n)


def test_reference_known_answers(oracle):
    # ptq1_0.rs:652-673
    src = np.zeros(128, np.float32)
    src[0], src[1], src[2], src[3], src[127] = -1.0, 1.0, 0.4, -0.4, 1.0
    blk = oracle.quantize_ptq1_0(src)
    assert blk.size == 28
    out = oracle.dequantize(GGML_PTQ1_0, blk, 128)
    assert out[0] == -1.0 and out[1] == 1.0 and out[2] == 0.0 and out[3] == 0.0 and out[4] == 0.0
    assert out[127] == 1.0
    # ptq1_0.rs:675-701: every byte pattern lands on {-1, 0, +1} * d
    data = np.array([(i * 37 + 11) & 0xFF for i in range(24)] + [0xAB, 0xC3, 0, 0], np.uint8)
    h = oracle.f32_to_f16(0.25)
    data[26], data[27] = h & 0xFF, h >> 8
    out = oracle.dequantize(GGML_PTQ1_0, data, 128)
    assert set(np.unique(out).tolist()) <= {-0.25, 0.0, 0.25}
    # ptq1_0.rs:737-756: all +1 weights; dot with all-ones activations is 128
    ones = np.ones(128, np.float32)
    w = oracle.quantize_ptq1_0(ones)
    assert np.all(oracle.dequantize(GGML_PTQ1_0, w, 128) == 1.0)
    a = oracle.quantize_q8_0(ones)
    assert abs(oracle.dot(GGML_PTQ1_0, w, a, 128) - 128.0) < 0.1


@pytest.mark.parametrize("n_blocks", [1, 3, 11, 32])
def test_dot_against_dequantized_and_integer(oracle, n_blocks):
    rng = np.random.default_rng(n_blocks)
    n = 128 * n_blocks
    w = rng.integers(0, 256, n_blocks * 28, dtype=np.uint8)
    for b in range(n_blocks):   # finite positive scales
        h = oracle.f32_to_f16(float(rng.uniform(0.01, 2.0)))
        w[b * 28 + 26], w[b * 28 + 27] = h & 0xFF, h >> 8
    a = oracle.quantize_q8_0(rng.standard_normal(n).astype(np.float32) * 3)
    got = oracle.dot(GGML_PTQ1_0, w, a, n)
    want = float(np.dot(oracle.dequantize(GGML_PTQ1_0, w, n).astype(np.float64),
                        oracle.dequantize(8, a, n).astype(np.float64)))
    assert abs(got - want) <= 1e-5 * max(1.0, abs(want))
    # unit scales: the dot is the exact integer sum of trit * int8
    one = oracle.f32_to_f16(1.0)
    w1, a1 = w.copy(), a.copy()
    for b in range(n_blocks):
        w1[b * 28 + 26], w1[b * 28 + 27] = one & 0xFF, one >> 8
    for s in range(n // 32):
        a1[s * 34], a1[s * 34 + 1] = one & 0xFF, one >> 8
    t = oracle.dequantize(GGML_PTQ1_0, w1, n).astype(np.int64)
    q = np.concatenate([a1[s * 34 + 2:s * 34 + 34].view(np.int8) for s in range(n // 32)]).astype(np.int64)
    assert oracle.dot(GGML_PTQ1_0, w1, a1, n) == float(np.dot(t, q))


def test_quantize_is_idempotent_on_dequantized(oracle):
    # the reference's LCG fixture (ptq1_0.rs:763-771) drives the weights
    seed = 0x12345678
    vals = []
    for _ in range(11 * 128):
        seed = (seed * 1664525 + 1013904223) & 0xFFFFFFFF
        vals.append(((seed >> 8) & 0xFFFF) / 32768.0 - 1.0)
    w = oracle.quantize_ptq1_0(np.array(vals, np.float32))
    deq = oracle.dequantize(GGML_PTQ1_0, w, w.size // 28 * 128)
    assert np.array_equal(oracle.quantize_ptq1_0(deq), w)


def test_synth_matches_q2_0_weights(oracle):
    rows, cols = 24, 512
    pt = oracle.synth_tensor(GGML_PTQ1_0, 9, "blk.0.ffn_up.weight", rows, cols, 0.02, 0.0)
    q2 = oracle.synth_tensor(GGML_Q2_0, 9, "blk.0.ffn_up.weight", rows, cols, 0.02, 0.0)
    assert pt.size == rows * cols // 128 * 28
    assert np.array_equal(oracle.dequantize(GGML_PTQ1_0, pt, rows * cols),
                          oracle.dequantize(GGML_Q2_0, q2, rows * cols))
