"""CPU pins of the oracle's f32 operators and greedy selection (ops.rs,
hearth-sampler lib.rs, qwen35.rs) via invariants, numpy brute force and the
reference tests' known answers."""
import ctypes as C

import numpy as np
import pytest


def _p(a):
    return a.ctypes.data


def test_rms_norm_unit_rms(oracle):
    lib = oracle.load()
    rng = np.random.default_rng(0)
    for n in (7, 128, 4096, 4100):
        x = rng.standard_normal(n).astype(np.float32) * 3
        w = np.ones(n, np.float32)
        out = np.zeros(n, np.float32)
        lib.ho_rms_norm(_p(x), _p(w), 1e-6, n, _p(out))
        assert abs(np.sqrt(np.mean(out.astype(np.float64) ** 2)) - 1.0) < 1e-5
        ref = x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6)
        assert np.allclose(out, ref, rtol=1e-5, atol=1e-6)


def test_rope_is_rotation(oracle):
    lib = oracle.load()
    max_seq, rd = 64, 128
    tab = np.zeros(max_seq * rd, np.float32)
    lib.ho_rope_table(max_seq, rd, 1e6, _p(tab))
    rng = np.random.default_rng(1)
    x = rng.standard_normal(128).astype(np.float32)
    for pos in (0, 1, 17, 63):
        y = x.copy()
        lib.ho_rope_apply(_p(tab), max_seq, rd, _p(y), pos)
        assert abs(np.linalg.norm(y) - np.linalg.norm(x)) < 1e-4
        half = rd // 2
        ang = pos * (1.0 / 1e6 ** (2.0 * np.arange(half) / rd))
        want0 = x[:half] * np.cos(ang) - x[half:] * np.sin(ang)
        want1 = x[:half] * np.sin(ang) + x[half:] * np.cos(ang)
        assert np.allclose(y, np.concatenate([want0, want1]), atol=2e-5)
    y = x.copy()
    lib.ho_rope_apply(_p(tab), max_seq, rd, _p(y), 0)
    assert np.array_equal(y, x)


def test_softmax_and_attention(oracle):
    lib = oracle.load()
    rng = np.random.default_rng(2)
    for n in (1, 5, 64, 2049):
        x = rng.standard_normal(n).astype(np.float32) * 4
        y = x.copy()
        lib.ho_softmax(_p(y), n)
        assert abs(y.astype(np.float64).sum() - 1.0) < 1e-5
        e = np.exp(x - x.max())
        assert np.allclose(y, e / e.sum(), rtol=1e-5, atol=1e-8)
    hd, seq = 128, 300
    q = rng.standard_normal(hd).astype(np.float32)
    k = rng.standard_normal((seq, hd)).astype(np.float32)
    v = rng.standard_normal((seq, hd)).astype(np.float32)
    out = np.zeros(hd, np.float32)
    scr = np.zeros(seq, np.float32)
    lib.ho_attention(_p(q), _p(k), _p(v), seq, hd, _p(out), _p(scr))
    s = k.astype(np.float64) @ q / np.sqrt(hd)
    p = np.exp(s - s.max())
    p /= p.sum()
    assert np.allclose(out, p @ v, rtol=1e-4, atol=1e-5)


def test_silu_known_answer(oracle):
    x = np.array([1.0, 0.0, -1.0], np.float32)
    oracle.load().ho_silu(_p(x), 3)
    assert abs(x[0] - 0.7310586) < 1e-6 and x[1] == 0.0   # ops.rs:1186-1190


def test_greedy_rules(oracle):
    lib = oracle.load()
    none = np.zeros(1, np.uint32)
    # hearth-sampler lib.rs:214-233 known answers
    for logits, want in (([-1.0, -2.0, 5.0, 0.5], 2), ([0.1, 0.2, 0.7, 0.05], 2)):
        a = np.array(logits, np.float32)
        assert lib.ho_sample_greedy_dense(_p(a), 4, _p(none), 0, 1.0) == want
    # ties: max_by keeps the LAST maximum; the qwen35 scan keeps the FIRST
    a = np.array([1.0, 3.0, 3.0, 2.0, 3.0], np.float32)
    assert lib.ho_sample_greedy_dense(_p(a.copy()), 5, _p(none), 0, 1.0) == 4
    assert lib.ho_argmax_first(_p(a), 5) == 1
    # repetition penalty: positive logits divided, negative multiplied, once per occurrence
    a = np.array([2.0, 2.1, -0.5, -0.4], np.float32)
    past = np.array([1, 1, 3], np.uint32)
    b = a.copy()
    tok = lib.ho_sample_greedy_dense(_p(b), 4, _p(past), 3, 1.1)
    assert tok == 0
    assert b[1] == np.float32(np.float32(2.1) / np.float32(1.1)) / np.float32(1.1)
    assert b[3] == np.float32(-0.4) * np.float32(1.1)
    # penalty 1.0 (within 1e-6) is a no-op
    b = a.copy()
    assert lib.ho_sample_greedy_dense(_p(b), 4, _p(past), 3, 1.0000001) == 1


def test_synth_generator_properties(oracle):
    lib = oracle.load()
    key = lib.ho_name_key(7, b"x")
    v = np.array([lib.ho_synth_int(key, i) for i in range(20000)], np.float64)
    assert abs(v.mean()) < 1500 and abs(v.std() / 37837.23 - 1) < 0.03
    # ternary: ~31% zeros (|w| < absmean/2 for a Gaussian), codes in {0,1,2}
    w = oracle.synth_tensor(42, 1, "t", 64, 1024, 0.02, 0.0)
    codes = np.stack([(w.reshape(-1, 34)[:, 2:] >> (2 * k)) & 3 for k in range(4)])
    frac0 = (codes == 1).mean()
    assert 0.28 < frac0 < 0.35 and not (codes == 3).any()
    # absmean scale: f16(sum|I| * c / 128)
    deq = oracle.dequantize(42, w, 64 * 1024)
    assert abs(np.abs(deq[deq != 0]).mean() / (0.02 * 0.7979) - 1) < 0.05
    # Q8_0 synth == quantize(float weights)
    q8 = oracle.synth_tensor(8, 1, "e", 2, 64, 0.02, 0.0)
    c = lib.ho_synth_scale(0.02)
    k2 = lib.ho_name_key(1, b"e")
    f = np.array([lib.ho_synth_int(k2, i) for i in range(128)], np.float32) * np.float32(c)
    assert np.array_equal(q8, oracle.quantize_q8_0(f))


def test_shared_exp_log_accuracy(oracle):
    """ho_exp / ho_log (the one exp/log both implementations use) against
    float64 numpy: exp within 2 ulp, log within 3 ulp of the correctly rounded value over the ranges
    the path feeds them (softmax and silu arguments, softplus of 1+e^x)."""
    lib = oracle.load()
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.uniform(-87.0, 88.0, 20000), rng.uniform(-20, 20, 20000),
                         np.array([0.0, -0.0, 1.0, -1.0, 1e-8, -1e-8, 88.7, -87.3])]).astype(np.float32)
    got = np.array([lib.ho_exp(float(x)) for x in xs], np.float32)
    want = np.exp(xs.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert (np.abs(got - want) / ulp).max() <= 2.0
    assert lib.ho_exp(-100.0) == 0.0 and np.isinf(lib.ho_exp(100.0))
    ys = np.concatenate([rng.uniform(1.0, 4.9e8, 20000), rng.uniform(1e-30, 10, 20000),
                         np.array([1.0, 2.0, 0.5, 1e-40, 3.4e38])]).astype(np.float32)
    got = np.array([lib.ho_log(float(y)) for y in ys], np.float32)
    want = np.log(ys.astype(np.float64))
    err = np.abs(got - want) / np.maximum(np.spacing(np.abs(want).astype(np.float32)), 1e-45)
    assert err.max() <= 3.0
    assert lib.ho_log(1.0) == 0.0


def test_device_order_matches_reference_order(oracle):
    """The device-order model (butterfly / split-sequence reductions) computes the
    same function as the reference-order model: identical greedy tokens on a tiny
    model and first-step logits within 1e-3; over longer runs the two diverge by
    Q8_0 rounding flips, the same effect as the reference's own scalar vs AVX2
    GEMV arms."""
    from hearth_amd.lib import ModelConfig, GGML_Q2_0
    cfg = ModelConfig(d_model=1024, n_layers=2, n_heads=8, n_kv_heads=4, head_dim=128, d_ffn=1024,
                      vocab=4096, max_seq=64, wtype=GGML_Q2_0)
    a = oracle.OracleModel(cfg, seed=3, threads=2, order=0)
    b = oracle.OracleModel(cfg, seed=3, threads=2, order=1)
    la, lb = a.forward(9, 0), b.forward(9, 0)
    assert np.abs(la - lb).max() / np.abs(la).max() < 1e-3
    # long attention: split-sequence vs single softmax on random data
    lib = oracle.load()
    rng = np.random.default_rng(4)
    hd, seq = 128, 2049
    q = rng.standard_normal(hd).astype(np.float32)
    k = rng.standard_normal((seq, hd)).astype(np.float32)
    v = rng.standard_normal((seq, hd)).astype(np.float32)
    s = k.astype(np.float64) @ q / np.sqrt(hd)
    p = np.exp(s - s.max())
    ref = (p / p.sum()) @ v
    out = np.zeros(hd, np.float32)
    scr = np.zeros(seq, np.float32)
    lib.ho_attention(q.ctypes.data, k.ctypes.data, v.ctypes.data, seq, hd, out.ctypes.data, scr.ctypes.data)
    assert np.allclose(out, ref, rtol=1e-4, atol=1e-5)


def test_device_order_attention_widths(oracle):
    """The device-order attention (the split kernels' grouping) against float64
    softmax attention at both chunk widths.  The width rule: 8192/hd positions
    per split, twice that once ceil(seq / (8192/hd)) * n_kv exceeds 256 (the
    MI355X CU count), checked against its closed form at the boundary."""
    lib = oracle.load()
    for hd, n_kv in ((128, 8), (256, 4), (128, 32)):
        c = 8192 // hd
        edge = c * (256 // n_kv)           # longest sequence on the narrow width
        assert lib.ho_attn_chunk(edge, hd, n_kv) == c
        assert lib.ho_attn_chunk(edge + 1, hd, n_kv) == 2 * c
        assert lib.ho_attn_chunk(1, hd, n_kv) == c
    rng = np.random.default_rng(8)
    for hd, n_kv, seq in ((128, 8, 2048), (128, 8, 2049), (128, 8, 2177), (256, 4, 2049), (256, 4, 300),
                          (128, 32, 600)):
        q = rng.standard_normal(hd).astype(np.float32)
        k = rng.standard_normal((seq, hd)).astype(np.float32)
        v = rng.standard_normal((seq, hd)).astype(np.float32)
        s = k.astype(np.float64) @ q / np.sqrt(hd)
        p = np.exp(s - s.max())
        ref = (p / p.sum()) @ v
        out = np.zeros(hd, np.float32)
        lib.ho_attention_dev(q.ctypes.data, k.ctypes.data, v.ctypes.data, seq, hd, n_kv, out.ctypes.data)
        assert np.allclose(out, ref, rtol=1e-4, atol=1e-5), (hd, n_kv, seq, np.abs(out - ref).max())
        # a dropped term breaks it: the same data one position shorter differs
        out2 = np.zeros(hd, np.float32)
        lib.ho_attention_dev(q.ctypes.data, k.ctypes.data, v.ctypes.data, seq - 1, hd, n_kv, out2.ctypes.data)
        assert not np.allclose(out2, ref, rtol=1e-4, atol=1e-5)
