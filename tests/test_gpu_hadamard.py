"""GPU parity of the qwen35 Hadamard fold (qwen35.rs:51-118, :532-620,
:881-970, :1054-1066, :1452-1478): every matmul input rotated by R = D.H
before Q8_0 (the GEMV's folded prologues and k_rot_q8_rows in the batched
prefill), the latent embedding's R^-1, ssm_out's grouped head order and the
tied head.  Logits and tokens must equal the device-order oracle bit for bit;
the oracle's fold is pinned by tests/test_oracle_hadamard.py."""
import os

import numpy as np
import pytest

from hearth_amd.lib import ModelConfig, GGML_Q2_0, GGML_PQ2_0, CONFIGS

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
HERE = os.path.dirname(os.path.abspath(__file__))

# fold widths 1024 (d, q heads 4 x 256, 8 v-heads x 128) and 2048 (ffn)
HYBH = ModelConfig(arch=1, d_model=1024, n_layers=4, n_heads=4, n_kv_heads=2, head_dim=256, rope_dim=64,
                   d_ffn=2048, vocab=4096, max_seq=128, wtype=GGML_Q2_0, full_attn_interval=2,
                   ssm_n_k_heads=2, ssm_n_v_heads=8, ssm_head_dim=128, ssm_conv_kernel=4, attn_out_gate=1,
                   had_block=1024, had_flags=3)


def signs_for(cfg, seed):
    rng = np.random.default_rng(seed)
    ws = sorted({cfg.d_model, cfg.d_ffn, cfg.n_heads * cfg.head_dim, cfg.ssm_n_v_heads * cfg.ssm_head_dim})
    return {w: rng.choice([-1.0, 1.0], w).astype(np.float32) for w in ws}


def make(ctx, oracle, cfg, seed, signs, env=None):
    from hearth_amd import Model
    old = {}
    for k, v in (env or {}).items():
        old[k] = os.environ.get(k)
        os.environ[k] = v
    try:
        m = Model(ctx, cfg)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    m.synthesize(seed)
    o = oracle.OracleModel(cfg, seed=seed, threads=16, order=oracle.OracleModel.DEVICE)
    for w, s in signs.items():
        m.set_hadamard_signs(w, s)
        o.set_signs(w, s)
    return m, o


@pytest.mark.parametrize("cfg", [HYBH, HYBH.replace(had_block=256, had_flags=0),
                                 HYBH.replace(had_flags=1, wtype=GGML_PQ2_0)],
                         ids=["b1024-latent-tied", "b256", "b1024-latent-pq2"])
def test_folded_decode_parity(ctx, oracle, cfg):
    signs = signs_for(cfg, 3)
    m, o = make(ctx, oracle, cfg, 11, signs)
    if cfg.had_flags & 2:
        assert "output.weight" not in [t[0] for t in m.tensors()]
    for pos, tok in enumerate([17, 400, 9, 4095, 0, 1234]):
        print(f"folded forward pos={pos}", flush=True)
        lg, _ = m.forward(tok, pos)
        lw = o.forward(tok, pos)
        assert np.array_equal(lg, lw), (pos, float(np.abs(lg - lw).max()))
    m.reset()
    o.reset()
    prompt = [5, 77, 1023, 4000]
    toks, lg = m.generate(prompt, 24, want_logits=True)
    tw, lw = o.generate(prompt, 24, want_logits=True)
    assert list(toks) == list(tw)
    assert np.array_equal(lg, lw)


@pytest.mark.parametrize("n_prompt", [3, 40])
def test_folded_batched_prefill(ctx, oracle, n_prompt):
    """The batched prefill (k_rot_q8_rows for every matmul input, the f32 hand-off
    of the GDN, attention and silu rows, the latent embedding rows) leaves the
    same state as the decode step fed token by token, and matches the oracle."""
    cfg = HYBH
    signs = signs_for(cfg, 5)
    prompt = [oracle.synth_token(9, i, cfg.vocab) for i in range(n_prompt)]
    mb, o = make(ctx, oracle, cfg, 13, signs, {"HH_BATCHED_PREFILL": "1"})
    mt, _ = make(ctx, oracle, cfg, 13, signs, {"HH_BATCHED_PREFILL": "0"})
    tb, lb = mb.generate(prompt, 8, want_logits=True)
    tt, lt = mt.generate(prompt, 8, want_logits=True)
    tw, lw = o.generate(prompt, 8, want_logits=True)
    assert list(tb) == list(tt) == list(tw)
    assert np.array_equal(lb, lt) and np.array_equal(lb, lw)


def test_folded_9b_slice(ctx, oracle):
    """9B geometry (d 4096, ffn 12288, 16 x 256 attention, 32 v-heads: rep 2),
    4 layers, block 1024, a 64-token batched prefill then 8 decode steps."""
    cfg = CONFIGS["9b-hybrid-q2"].replace(n_layers=4, max_seq=256, had_block=1024, had_flags=1)
    signs = signs_for(cfg, 7)
    m, o = make(ctx, oracle, cfg, 21, signs)
    prompt = [oracle.synth_token(4, i, cfg.vocab) for i in range(64)]
    toks, lg = m.generate(prompt, 8, want_logits=True)
    tw, lw = o.generate(prompt, 8, want_logits=True)
    assert list(toks) == list(tw)
    assert np.array_equal(lg, lw)


def test_folded_gguf_roundtrip(ctx, oracle, tmp_path):
    """A folded, tied, latent model written as GGUF with prism.hadamard.* and
    loaded by hh_model_load_gguf decodes like the model it came from."""
    import sys
    sys.path.insert(0, HERE)
    import gguf_writer as gw
    from hearth_amd import Model
    cfg = HYBH
    signs = signs_for(cfg, 8)
    m, _ = make(ctx, oracle, cfg, 31, signs)
    tensors = []
    for name, t, ne0, ne1, nb in m.tensors():
        data = m.download(name, nb).tobytes()
        shape = (ne0,) if ne1 == 1 and t == 0 else (ne0, ne1)
        tensors.append((name, t, shape, data))
    meta = gw.model_meta(cfg) + gw.hadamard_meta(cfg.had_block, signs, version=2, latent=True, tied=True)
    p = tmp_path / "folded.gguf"
    gw.write_gguf(str(p), meta, tensors)
    g = Model.from_gguf(ctx, str(p), ctx_cap=cfg.max_seq)
    assert g.cfg.had_block == cfg.had_block and g.cfg.had_flags == 3
    prompt = [7, 8, 9, 10]
    ta, la = m.generate(prompt, 12, want_logits=True)
    tb, lb = g.generate(prompt, 12, want_logits=True)
    assert list(ta) == list(tb) and np.array_equal(la, lb)
    g.close()
    m.close()


def test_folded_errors(ctx):
    from hearth_amd import Model, HHError
    with pytest.raises(HHError):     # a width that is not whole fold chunks
        Model(ctx, HYBH.replace(had_block=4096))
    with pytest.raises(HHError):     # the fold is a qwen35 feature
        Model(ctx, ModelConfig(d_model=1024, n_layers=1, n_heads=8, n_kv_heads=4, head_dim=128, d_ffn=1024,
                               vocab=4096, max_seq=64, wtype=GGML_Q2_0, had_block=1024))
    m = Model(ctx, HYBH)
    with pytest.raises(HHError):
        m.set_hadamard_signs(1024, np.full(1024, 0.5, np.float32))
    m.set_hadamard_signs(3072, np.ones(3072, np.float32))   # a width the model does not fold: ignored
    m.close()
