"""Pins the oracle's Hadamard fold (qwen35.rs:51-118 walsh_hadamard_in_place /
hadamard_rotate / hadamard_unrotate, the folded matmuls of qwen35.rs:881-970,
the latent embedding of :1054-1066, the grouped ssm_out input of :1452-1478
and the tied head of :532-620) against scipy's Sylvester Hadamard matrix and
a float64 numpy restatement of a folded hybrid (tests/np_hybrid.py)."""
import numpy as np
import pytest
import scipy.linalg

from hearth_amd.lib import ModelConfig, GGML_Q2_0
from np_hybrid import NpHybrid

TOL = 1e-3


@pytest.mark.parametrize("n", [2, 4, 8, 64, 256, 512, 1024])
def test_wht_matches_sylvester_matrix(oracle, n):
    """The butterfly equals H_n / sqrt(n) (scipy.linalg.hadamard, Sylvester order)."""
    x = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    want = scipy.linalg.hadamard(n).astype(np.float64) @ x.astype(np.float64) / np.sqrt(n)
    got = oracle.wht(x)
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()


def test_wht_known_answers(oracle):
    """e_0 -> every entry 1/sqrt(n); all-ones -> sqrt(n) e_0 (exact at n = 1024,
    where 1/sqrt(n) = 1/32); the normalized transform is an involution."""
    n = 1024
    e0 = np.zeros(n, np.float32)
    e0[0] = 1
    assert np.array_equal(oracle.wht(e0), np.full(n, 1 / 32, np.float32))
    want = np.zeros(n, np.float32)
    want[0] = 32
    assert np.array_equal(oracle.wht(np.ones(n, np.float32)), want)
    x = np.random.default_rng(1).standard_normal(n).astype(np.float32)
    assert np.abs(oracle.wht(oracle.wht(x)) - x).max() < 1e-5


def test_rotate_unrotate_order(oracle):
    """rotate = WHT(signs * x) per block; unrotate = signs * WHT(x); they invert
    each other, and swapping the order is a different map."""
    rng = np.random.default_rng(2)
    n, b = 2048, 512
    x = rng.standard_normal(n).astype(np.float32)
    s = rng.choice([-1.0, 1.0], n).astype(np.float32)
    H = scipy.linalg.hadamard(b) / np.sqrt(b)
    r = oracle.hadamard_rotate(x, s, b)
    want = ((x * s).astype(np.float64).reshape(-1, b) @ H.T).reshape(-1)
    assert np.abs(r - want).max() < 1e-5
    u = oracle.hadamard_rotate(r, s, b, inverse=True)
    assert np.abs(u - x).max() < 1e-5
    wrong = oracle.hadamard_rotate(r, s, b)   # R R x != x
    assert np.abs(wrong - x).max() > 0.1
    # a vector shorter than the block gets the sign pass only (chunks_exact)
    short = rng.standard_normal(256).astype(np.float32)
    ss = rng.choice([-1.0, 1.0], 256).astype(np.float32)
    assert np.array_equal(oracle.hadamard_rotate(short, ss, 1024), short * ss)


# d 1024, q heads 4 x 256 = 1024, 8 v-heads x 128 = 1024 (rep 4), ffn 2048:
# fold widths 1024 and 2048
HYBH = ModelConfig(arch=1, d_model=1024, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=256, rope_dim=64,
                   d_ffn=2048, vocab=4096, max_seq=64, wtype=GGML_Q2_0, full_attn_interval=2,
                   ssm_n_k_heads=2, ssm_n_v_heads=8, ssm_head_dim=128, ssm_conv_kernel=4, attn_out_gate=1,
                   had_block=1024, had_flags=3)
TOKENS = [11, 905, 42, 3071]


def fold_signs(seed, widths):
    rng = np.random.default_rng(seed)
    return {w: rng.choice([-1.0, 1.0], w).astype(np.float32) for w in widths}


def folded(oracle, cfg, seed, signs, order=0):
    m = oracle.OracleModel(cfg, seed=seed, threads=2, order=order)
    for w, s in signs.items():
        m.set_signs(w, s)
    return m


@pytest.mark.parametrize("cfg", [HYBH, HYBH.replace(had_block=256, had_flags=0)], ids=["b1024-latent-tied", "b256"])
def test_folded_hybrid_matches_numpy(oracle, cfg):
    signs = fold_signs(3, [1024, 2048])
    m = folded(oracle, cfg, 17, signs)
    if cfg.had_flags & 2:
        with pytest.raises(KeyError):
            m.tensor("output.weight")
    out = [m.forward(t, p) for p, t in enumerate(TOKENS)]
    ref = NpHybrid(m, cfg, signs=signs)
    want = [ref.forward(t, p) for p, t in enumerate(TOKENS)]
    errs = [float(np.abs(o - w).max() / np.abs(w).max()) for o, w in zip(out, want)]
    assert max(errs) < TOL, errs
    # the fold changes the model: the unfolded model's logits differ
    plain = oracle.OracleModel(cfg.replace(had_block=0, had_flags=cfg.had_flags & 2), seed=17, threads=2)
    if cfg.had_flags & 2:
        return
    assert np.abs(plain.forward(TOKENS[0], 0) - out[0]).max() > 20 * TOL * np.abs(out[0]).max()


@pytest.mark.parametrize("mutation", ["no_ssm_perm", "unrotate_as_rotate"])
def test_folded_hybrid_detects_mutation(oracle, mutation):
    signs = fold_signs(3, [1024, 2048])
    m = folded(oracle, HYBH, 17, signs)
    out = [m.forward(t, p) for p, t in enumerate(TOKENS)]
    bad = NpHybrid(m, HYBH, mutate=mutation, signs=signs)
    errs = [float(np.abs(o - bad.forward(t, p)).max() / np.abs(o).max()) for o, (p, t) in zip(out, enumerate(TOKENS))]
    assert max(errs) > 20 * TOL, (mutation, errs)


def test_folded_device_order_close(oracle):
    signs = fold_signs(5, [1024, 2048])
    a = folded(oracle, HYBH, 9, signs, order=0)
    b = folded(oracle, HYBH, 9, signs, order=1)
    for p, t in enumerate(TOKENS):
        la, lb = a.forward(t, p), b.forward(t, p)
        assert np.abs(la - lb).max() <= 1e-4 * np.abs(la).max() + 1e-6
