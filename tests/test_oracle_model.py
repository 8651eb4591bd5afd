"""CPU checks of the oracle's model composition on tiny geometries."""
import numpy as np
import pytest

from hearth_amd.lib import ModelConfig, GGML_Q1_0, GGML_Q2_0

TINY = ModelConfig(d_model=1024, n_layers=2, n_heads=8, n_kv_heads=4, head_dim=128, d_ffn=1024,
                   vocab=4096, max_seq=64, wtype=GGML_Q2_0)
TINY_HYB = ModelConfig(arch=1, d_model=1024, n_layers=4, n_heads=4, n_kv_heads=2, head_dim=256, rope_dim=64,
                       d_ffn=1024, vocab=4096, max_seq=64, wtype=GGML_Q2_0, full_attn_interval=4,
                       ssm_n_k_heads=2, ssm_n_v_heads=4, ssm_head_dim=128, ssm_conv_kernel=4,
                       attn_out_gate=1)


def test_tiny_dense_deterministic(oracle):
    m = oracle.OracleModel(TINY, seed=3, threads=2)
    t1, l1 = m.generate([1, 2, 3], 8, want_logits=True)
    m.reset()
    t2, l2 = m.generate([1, 2, 3], 8, want_logits=True)
    assert np.array_equal(t1, t2) and np.array_equal(l1, l2)
    assert np.isfinite(l1).all() and l1.std() > 0.1


def test_tiny_dense_first_step_by_hand(oracle):
    """Layer-by-layer numpy restatement of mod.rs:451-860 for one token at pos 0
    (seq_len 1 makes attention the identity on v), built from the oracle's
    dequantized tensors: logits agree to 1e-3 relative."""
    from tests.fixtures import np_dequant
    cfg = TINY.replace(n_layers=1)
    m = oracle.OracleModel(cfg, seed=5, threads=2)
    logits = m.forward(7, 0)
    d, hd, nh, nkv = cfg.d_model, cfg.head_dim, cfg.n_heads, cfg.n_kv_heads

    def W(name, rows, cols, t=GGML_Q2_0):
        return np_dequant(t, m.tensor(name), rows * cols).reshape(rows, cols).astype(np.float64)

    def F(name):
        return m.tensor(name).view(np.float32).astype(np.float64)

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x) + cfg.eps) * w

    def q8(x):
        return np_dequant(8, oracle.quantize_q8_0(x.astype(np.float32)), x.size).astype(np.float64)

    h = np_dequant(8, m.tensor("token_embd.weight"), cfg.vocab * d).reshape(cfg.vocab, d)[7].astype(np.float64)
    x = q8(rms(h, F("blk.0.attn_norm.weight")))
    v = W("blk.0.attn_v.weight", nkv * hd, d) @ x
    # one position: softmax weight 1 -> attention output = v of the kv head
    att = np.concatenate([v[(qh // (nh // nkv)) * hd:(qh // (nh // nkv) + 1) * hd] for qh in range(nh)])
    h = h + W("blk.0.attn_output.weight", d, nh * hd) @ q8(att)
    x = q8(rms(h, F("blk.0.ffn_norm.weight")))
    g = W("blk.0.ffn_gate.weight", cfg.d_ffn, d) @ x
    u = W("blk.0.ffn_up.weight", cfg.d_ffn, d) @ x
    h = h + W("blk.0.ffn_down.weight", d, cfg.d_ffn) @ q8(g / (1 + np.exp(-g)) * u)
    x = q8(rms(h, F("output_norm.weight")))
    want = np_dequant(8, m.tensor("output.weight"), cfg.vocab * d).reshape(cfg.vocab, d).astype(np.float64) @ x
    err = np.abs(logits - want).max() / np.abs(want).max()
    assert err < 1e-3, err


def test_kv_prefill_values_are_f16(oracle):
    cfg = TINY.replace(max_seq=32)
    m = oracle.OracleModel(cfg, seed=1, threads=1)
    m.prefill_kv_synthetic(9, 16)
    logits = m.forward(5, 16)
    assert np.isfinite(logits).all()


def test_tiny_hybrid_runs(oracle):
    m = oracle.OracleModel(TINY_HYB, seed=4, threads=2)
    toks, logits = m.generate([3, 4, 5, 6], 6, want_logits=True)
    assert np.isfinite(logits).all() and logits.std() > 0.05
    m.reset()
    toks2, _ = m.generate([3, 4, 5, 6], 6)
    assert np.array_equal(toks, toks2)


def test_gdn_single_step_closed_form(oracle):
    """qwen35.rs:1239-1492 from a zero state and zero conv history: the window is
    [0,..,0,x] so conv_out = w[ch][K-1] x[ch]; one delta-rule step gives
    S = k (beta v)^T and o = beta v (k.q) / sqrt(hd).  A numpy restatement of the
    whole 1-layer hybrid (GDN layer, FFN, head) matches the oracle's logits."""
    from tests.fixtures import np_dequant
    cfg = TINY_HYB.replace(n_layers=1, full_attn_interval=2)
    m = oracle.OracleModel(cfg, seed=8, threads=1)
    tok = 11
    logits = m.forward(tok, 0)
    d, hd = cfg.d_model, cfg.ssm_head_dim
    nk, nv = cfg.ssm_n_k_heads, cfg.ssm_n_v_heads
    kdim, vdim = nk * hd, nv * hd
    conv_dim = 2 * kdim + vdim
    K = cfg.ssm_conv_kernel

    def W(name, rows, cols):
        return np_dequant(cfg.wtype, m.tensor(name), rows * cols).reshape(rows, cols).astype(np.float64)

    def F(name):
        return m.tensor(name).view(np.float32).astype(np.float64)

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x) + cfg.eps) * w

    def q8(x):
        return np_dequant(8, oracle.quantize_q8_0(x.astype(np.float32)), x.size).astype(np.float64)

    silu = lambda z: z / (1 + np.exp(-z))
    h = np_dequant(8, m.tensor("token_embd.weight"), cfg.vocab * d).reshape(cfg.vocab, d)[tok].astype(np.float64)
    nrm = rms(h, F("blk.0.attn_norm.weight"))
    x = q8(nrm)
    qkv = W("blk.0.attn_qkv.weight", conv_dim, d) @ x
    z = W("blk.0.attn_gate.weight", vdim, d) @ x
    a = F("blk.0.ssm_alpha.weight").reshape(nv, d) @ nrm
    b = F("blk.0.ssm_beta.weight").reshape(nv, d) @ nrm
    conv = F("blk.0.ssm_conv1d.weight").reshape(conv_dim, K)[:, K - 1] * qkv
    co = silu(conv)
    qh = co[:kdim].reshape(nk, hd)
    kh = co[kdim:2 * kdim].reshape(nk, hd)
    qh = qh / np.sqrt((qh * qh).sum(1, keepdims=True) + cfg.eps)
    kh = kh / np.sqrt((kh * kh).sum(1, keepdims=True) + cfg.eps)
    v = co[2 * kdim:].reshape(nv, hd)
    beta = 1 / (1 + np.exp(-b))
    o = np.stack([beta[h_] * v[h_] * (kh[h_ % nk] @ qh[h_ % nk]) / np.sqrt(hd) for h_ in range(nv)])
    on = np.stack([rms(o[h_], F("blk.0.ssm_norm.weight")) for h_ in range(nv)]).reshape(-1) * silu(z)
    h = h + W("blk.0.ssm_out.weight", d, vdim) @ q8(on)
    x = q8(rms(h, F("blk.0.post_attention_norm.weight")))
    g = W("blk.0.ffn_gate.weight", cfg.d_ffn, d) @ x
    u = W("blk.0.ffn_up.weight", cfg.d_ffn, d) @ x
    h = h + W("blk.0.ffn_down.weight", d, cfg.d_ffn) @ q8(silu(g) * u)
    x = q8(rms(h, F("output_norm.weight")))
    want = np_dequant(8, m.tensor("output.weight"), cfg.vocab * d).reshape(cfg.vocab, d).astype(np.float64) @ x
    err = np.abs(logits - want).max() / np.abs(want).max()
    assert err < 1e-3, err
