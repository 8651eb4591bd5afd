"""Pins the oracle's qwen35 hybrid layers (qwen35.rs:1239-1640) against an
independent float64 numpy restatement (tests/np_hybrid.py) over several decode
steps, so that the multi-step Gated-DeltaNet recurrence (state decay, the
v - S^T k term on the undecayed state, the conv window shift) and the gated
full-attention layer ([q_h | gate_h] interleave, head norms at hd 256, partial
RoPE, o / (1 + e^-gate)) are checked, not only the zero-state first step.

Each test also runs the numpy restatement with one deliberate mistake and
asserts that the oracle is far from it: the comparison can tell each plausible
error apart from the right rule."""
import numpy as np
import pytest

from hearth_amd.lib import ModelConfig, GGML_Q2_0
from np_hybrid import NpHybrid

# layer 0: Gated-DeltaNet, layer 1: gated full attention (full_attn_interval 2);
# 2 k-groups, 4 v-heads (rep 2: h % n_groups differs from h // rep)
HYB2 = ModelConfig(arch=1, d_model=1024, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=256, rope_dim=64,
                   d_ffn=1024, vocab=4096, max_seq=64, wtype=GGML_Q2_0, full_attn_interval=2,
                   ssm_n_k_heads=2, ssm_n_v_heads=4, ssm_head_dim=128, ssm_conv_kernel=4, attn_out_gate=1)
TOKENS = [11, 905, 42, 3071, 7]
TOL = 1e-3


def _rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / np.abs(b).max())


def _run(np_model, toks):
    np_model.reset()
    return [np_model.forward(t, p) for p, t in enumerate(toks)]


@pytest.fixture(scope="module")
def hyb(oracle):
    m = oracle.OracleModel(HYB2, seed=21, threads=2)
    out = {}
    for order in (oracle.OracleModel.REFERENCE, oracle.OracleModel.DEVICE):
        m.set_order(order)
        m.reset()
        out[order] = [m.forward(t, p) for p, t in enumerate(TOKENS)]
    m.set_order(oracle.OracleModel.REFERENCE)
    return m, out


def test_hybrid_multistep_matches_numpy(hyb, oracle):
    """Five tokens through [GDN, gated attention]: every step's logits, in both
    the reference order and the device order, are within 1e-3 of float64."""
    m, out = hyb
    want = _run(NpHybrid(m, HYB2), TOKENS)
    for order in out:
        errs = [_rel(o, w) for o, w in zip(out[order], want)]
        assert max(errs) < TOL, (order, errs)


@pytest.mark.parametrize("mutation", ["decay_before_dot", "state_transposed", "gate_from_q",
                                      "no_conv_history", "khead_div", "rope_full", "no_qk_norm"])
def test_hybrid_numpy_detects_mutation(hyb, mutation):
    """The same comparison with one plausible mistake in the restatement misses
    by far more than the tolerance at some step."""
    m, out = hyb
    bad = _run(NpHybrid(m, HYB2, mutate=mutation), TOKENS)
    errs = [_rel(o, w) for o, w in zip(out[0], bad)]
    assert max(errs) > 20 * TOL, (mutation, errs)


def test_gdn_two_step_closed_form(oracle):
    """Two delta-rule steps from the zero state, written out (qwen35.rs:1371-1404):
    S1 = k1 (b1 v1)^T; dot2 = b1 v1 (k1.k2) on the undecayed S1;
    S2 = e^g2 S1 + k2 b2 (v2 - dot2)^T; o2 = S2^T q2 / sqrt(hd).
    Evaluated on random unit k/q and checked against the loop form used by the
    numpy restatement, so the restatement's loop is itself pinned."""
    rng = np.random.default_rng(5)
    hd = 128
    unit = lambda x: x / np.linalg.norm(x)
    k1, k2, q2 = (unit(rng.standard_normal(hd)) for _ in range(3))
    v1, v2 = rng.standard_normal(hd), rng.standard_normal(hd)
    b1, b2, g2 = 0.7, 0.4, -0.69
    S1 = np.outer(k1, b1 * v1)
    dot2 = b1 * v1 * (k1 @ k2)
    S2 = np.exp(g2) * S1 + np.outer(k2, b2 * (v2 - dot2))
    o2 = S2.T @ q2 / np.sqrt(hd)
    # loop form, as in qwen35.rs: per column j, dot then update
    S = np.zeros((hd, hd))
    for k, v, b, g in ((k1, v1, b1, 0.0), (k2, v2, b2, g2)):
        for j in range(hd):
            dot = sum(S[i, j] * k[i] for i in range(hd))
            bd = b * (v[j] - dot)
            for i in range(hd):
                S[i, j] = S[i, j] * np.exp(g) + k[i] * bd
    o = np.array([sum(S[i, j] * q2[i] for i in range(hd)) for j in range(hd)]) / np.sqrt(hd)
    assert np.allclose(S, S2, rtol=0, atol=1e-12) and np.allclose(o, o2, rtol=0, atol=1e-12)
    # decay before the dot gives a different o2 (by ~|1-e^g| b1 b2 (k1.k2)^2 terms)
    S2_bad = np.exp(g2) * S1 + np.outer(k2, b2 * (v2 - np.exp(g2) * dot2))
    assert np.abs(S2_bad.T @ q2 / np.sqrt(hd) - o2).max() > 1e-4


def test_gated_attention_pos0_is_gated_v(oracle):
    """One gated full-attention layer at pos 0: softmax over one position is 1,
    so the attention output of q head h is v of its kv head times
    sigmoid(gate_h), gate_h being the second half of head h's 2*hd block of
    attn_q (qwen35.rs:1526-1560, :1627-1629)."""
    cfg = HYB2.replace(n_layers=1, full_attn_interval=1)
    m = oracle.OracleModel(cfg, seed=4, threads=2)
    logits = m.forward(77, 0)
    ref = NpHybrid(m, cfg)
    # written out without the restatement's attention code
    d, hd, nh, nkv = cfg.d_model, cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    h = ref.W("token_embd.weight", cfg.vocab, d, 8)[77]
    x = ref.q8(ref.rms(h, ref.F("blk.0.attn_norm.weight")))
    qg = ref.W("blk.0.attn_q.weight", 2 * nh * hd, d) @ x
    v = ref.W("blk.0.attn_v.weight", nkv * hd, d) @ x
    att = np.concatenate([v[(qh // (nh // nkv)) * hd:][:hd] / (1 + np.exp(-qg[qh * 2 * hd + hd:][:hd]))
                          for qh in range(nh)])
    h = h + ref.W("blk.0.attn_output.weight", d, nh * hd) @ ref.q8(att)
    x = ref.q8(ref.rms(h, ref.F("blk.0.post_attention_norm.weight")))
    g = ref.W("blk.0.ffn_gate.weight", cfg.d_ffn, d) @ x
    u = ref.W("blk.0.ffn_up.weight", cfg.d_ffn, d) @ x
    h = h + ref.W("blk.0.ffn_down.weight", d, cfg.d_ffn) @ ref.q8(ref.silu(g) * u)
    want = ref.W("output.weight", cfg.vocab, d, 8) @ ref.q8(ref.rms(h, ref.F("output_norm.weight")))
    assert _rel(logits, want) < TOL
    assert _rel(logits, ref.forward(77, 0)) < TOL


def test_hybrid_device_order_matches_reference_order(hyb):
    """The oracle's two fp32 association orders agree within 1e-4 on every
    step of the hybrid (the dense counterpart is in test_oracle_ops.py)."""
    _, out = hyb
    errs = [_rel(a, b) for a, b in zip(out[1], out[0])]
    assert max(errs) < 1e-4, errs


@pytest.mark.parametrize("seed", [2026, 7, 99])
def test_hybrid_device_order_tokens_vs_reference_order(oracle, seed):
    """32 greedy tokens of the 4-layer hybrid, teacher-forced on the
    reference-order oracle's own sequence: the device-order oracle (which the
    HIP library equals bit for bit) picks the same token at every step, or the
    two tokens are closer in the reference logits than the reference's scalar
    and AVX2 arms differ (tests/tokcheck.py)."""
    import sys, os
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import make_golden
    from tokcheck import reference_run, check_candidate, ambiguous_steps
    cfg = make_golden.HYBRID
    seq, ref_logits, spread = reference_run(oracle, cfg, seed, make_golden.PROMPT, 32)
    dev = oracle.OracleModel(cfg, seed=seed, threads=4, order=oracle.OracleModel.DEVICE)
    div = check_candidate(cfg, seq, ref_logits, spread, len(make_golden.PROMPT), dev.forward)
    amb = ambiguous_steps(ref_logits, spread)
    print(f"seed {seed}: arm spread {spread:.3g}, ambiguous steps {amb}, "
          f"AVX2-arm divergences {reference_run.avx_divergences}, divergences {div}", flush=True)
    assert len(div) <= amb


def _delta_sequential(S, K, Q, V, g, beta):
    """qwen35.rs:1371-1404 token by token in float64 (dot on the undecayed state)."""
    S = S.copy()
    out = []
    for t in range(len(g)):
        dot = S.T @ K[t]
        S = S * np.exp(g[t]) + np.outer(K[t], beta[t] * (V[t] - dot))
        out.append(S.T @ Q[t] / np.sqrt(S.shape[0]))
    return S, np.array(out)


def _delta_chunked(S, K, Q, V, g, beta, C):
    """The chunked form the device's hh_gdn_chunk.hip evaluates (its header):
    per chunk, G = cumsum g; (I + A) U = B with A[t][s] = beta_t e^{G_{t-1}-G_s} k_t.k_s;
    o_t = e^{G_t} S^T q_t + sum_{s<=t} e^{G_t-G_s} (q_t.k_s) u_s; S' = e^{G_last} S + sum e^{G_last-G_s} k_s u_s^T."""
    S = S.copy()
    outs = []
    hd = S.shape[0]
    for c0 in range(0, len(g), C):
        k, q, v, gg, b = K[c0:c0 + C], Q[c0:c0 + C], V[c0:c0 + C], g[c0:c0 + C], beta[c0:c0 + C]
        n = len(gg)
        G = np.cumsum(gg)
        Gm1 = np.concatenate([[0.0], G[:-1]])
        A = np.zeros((n, n))
        for t in range(n):
            for s in range(t):
                A[t, s] = b[t] * np.exp(Gm1[t] - G[s]) * (k[t] @ k[s])
        B = b[:, None] * (v - np.exp(Gm1)[:, None] * (k @ S))
        U = np.linalg.solve(np.eye(n) + A, B)
        M = np.tril(np.exp(G[:, None] - G[None, :]) * (q @ k.T))
        outs.append((np.exp(G)[:, None] * (q @ S) + M @ U) / np.sqrt(hd))
        S = np.exp(G[-1]) * S + (k * np.exp(G[-1] - G)[:, None]).T @ U
    return S, np.concatenate(outs)


@pytest.mark.parametrize("n_tok", [1, 63, 64, 150])
def test_chunked_delta_rule_equals_sequential(n_tok):
    """The chunked restatement of the delta rule (the algebra of the device's
    optional chunked prefill) equals the token-by-token rule in float64, from a
    nonzero state, across chunk boundaries and a ragged last chunk."""
    rng = np.random.default_rng(n_tok)
    hd = 32
    unit = lambda x: x / np.linalg.norm(x, axis=1, keepdims=True)
    K, Q = unit(rng.standard_normal((n_tok, hd))), unit(rng.standard_normal((n_tok, hd)))
    V = rng.standard_normal((n_tok, hd))
    g = -np.log1p(np.exp(rng.standard_normal(n_tok)))        # softplus(.) * (-1)
    beta = 1 / (1 + np.exp(-rng.standard_normal(n_tok)))
    S0 = rng.standard_normal((hd, hd)) * 0.1
    Ss, Os = _delta_sequential(S0, K, Q, V, g, beta)
    Sc, Oc = _delta_chunked(S0, K, Q, V, g, beta, 64)
    assert np.abs(Sc - Ss).max() < 1e-10 and np.abs(Oc - Os).max() < 1e-10
    # dropping the decay from the dot term (a plausible slip) is visible
    Sb, _ = _delta_chunked(S0, K, Q, V, np.zeros_like(g), beta, 64)
    assert n_tok == 1 or np.abs(Sb - Ss).max() > 1e-3
