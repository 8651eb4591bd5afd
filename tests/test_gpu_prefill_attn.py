"""Batched-prefill attention (forward_batch's per-token attention, mod.rs:1101-1140
over ops.rs:353-406) through hh_attention_prefill, against a float64 numpy
restatement of causal softmax attention:

  * mode 0, the split/merge kernels the batched prefill runs by default: within
    1e-5 of float64, and each token's row equal bit for bit to the decode
    operator hh_attention at seq_len pos0 + t + 1 (the prefill restates the
    decode order);
  * mode 1, the fp32-MFMA flash form (HH_PREFILL_ATTN=mfma): within 1e-5 of
    float64 (its sums are regrouped, so this is its parity bar).

Geometries cover head_dim 128 and 256, query groups 1, 3, 4, 6 and 8 (so the
MFMA kernel's 1-4 token tiles per workgroup), partial 16-token tiles, a
prompt that starts past position 0 and one long enough for many chunks.  A
model-level check runs a 9B-shaped slice and an 8B-shaped slice through the
batched prefill both ways."""
import os

import numpy as np
import pytest

from hearth_amd.lib import CONFIGS

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _ref(q, k, v, pos0):
    n, nh, hd = q.shape
    nkv = k.shape[0]
    G = nh // nkv
    out = np.zeros((n, nh, hd))
    for t in range(n):
        L = pos0 + t + 1
        for h in range(nh):
            kk = k[h // G, :L].astype(np.float64)
            s = kk @ q[t, h].astype(np.float64) / np.sqrt(hd)
            p = np.exp(s - s.max())
            out[t, h] = (p / p.sum()) @ v[h // G, :L].astype(np.float64)
    return out


@pytest.mark.parametrize("nh,nkv,hd,pos0,n", [(32, 8, 128, 0, 300), (16, 4, 256, 37, 70), (16, 2, 128, 5, 50),
                                              (8, 8, 128, 0, 45), (24, 4, 256, 0, 33), (6, 2, 128, 100, 29)])
def test_prefill_attention_modes_vs_float64(ctx, nh, nkv, hd, pos0, n):
    rng = np.random.default_rng(nh * 1000 + hd + pos0 + n)
    ms = pos0 + n + 24
    q = rng.standard_normal((n, nh, hd)).astype(np.float32)
    k = rng.standard_normal((nkv, ms, hd)).astype(np.float32)
    v = rng.standard_normal((nkv, ms, hd)).astype(np.float32)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    dq, dk, dv = dev(q), dev(k), dev(v)
    want = _ref(q, k, v, pos0)
    print(f"prefill attention {nh}/{nkv} x {hd}, pos0 {pos0}, {n} tokens", flush=True)
    got = {}
    for mode in (0, 1):
        out = torch.full((n * nh * hd,), float("nan"), dtype=torch.float32, device="cuda")
        ctx.attention_prefill(dq, dk, dv, nh, nkv, hd, ms, pos0, n, mode, out)
        ctx.sync()
        got[mode] = out.cpu().numpy().reshape(n, nh, hd)
        err = float(np.abs(got[mode] - want).max() / np.abs(want).max())
        print(f"  mode {mode}: max rel err vs float64 {err:.2e}", flush=True)
        assert np.isfinite(got[mode]).all() and err < 1e-5, (mode, err)
    # the default path is the decode operator's order, token by token
    for t in sorted({0, n // 2, n - 1}):
        one = torch.zeros(nh * hd, dtype=torch.float32, device="cuda")
        ctx.attention(dev(q[t]), dk, dv, nh, nkv, hd, ms, pos0 + t + 1, one)
        ctx.sync()
        assert np.array_equal(one.cpu().numpy(), got[0][t].reshape(-1)), t


def _model_env(ctx, cfg, seed, env):
    from hearth_amd import Model
    old = os.environ.get("HH_PREFILL_ATTN")
    if env:
        os.environ["HH_PREFILL_ATTN"] = env
    else:
        os.environ.pop("HH_PREFILL_ATTN", None)
    try:
        m = Model(ctx, cfg)
    finally:
        if old is None:
            os.environ.pop("HH_PREFILL_ATTN", None)
        else:
            os.environ["HH_PREFILL_ATTN"] = old
    m.synthesize(seed)
    return m


@pytest.mark.parametrize("name,kv_type", [("9b-hybrid-q2", 0), ("8b-q2", 0), ("8b-q2", 8)])
def test_mfma_prefill_model_logits(ctx, oracle, name, kv_type):
    """The same prompt prefilled with the default attention and with the MFMA
    form: the first generated token's logits within 5e-2 relative (each
    regrouped sum can flip a later Q8_0 rounding, as the reference's own scalar
    and AVX2 arms do to each other)."""
    cfg = CONFIGS[name].replace(n_layers=2 if name == "8b-q2" else 8, max_seq=640, kv_type=kv_type)
    prompt = [oracle.synth_token(12, i, cfg.vocab) for i in range(300)]
    res = []
    for env in (None, "mfma"):
        m = _model_env(ctx, cfg, 41, env)
        m.prefill(prompt[:-1], 0)
        lg, _ = m.forward(prompt[-1], len(prompt) - 1)
        res.append(lg.astype(np.float64))
        m.close()
    err = float(np.abs(res[0] - res[1]).max() / np.abs(res[0]).max())
    print(f"{name} kv{kv_type}: logits rel err MFMA vs default prefill attention {err:.2e}", flush=True)
    assert np.isfinite(res[1]).all() and err < 5e-2, err


def test_attention_prefill_errors(ctx):
    from hearth_amd import HHError
    z = torch.zeros(16 * 4 * 128 * 64, dtype=torch.float32, device="cuda")
    cases = [((16, 4, 128, 64, 0, 16, 2), 1),      # mode
             ((16, 4, 128, 64, 60, 8, 0), 7),      # past max_seq
             ((16, 4, 96, 64, 0, 8, 1), 3),        # head_dim
             ((18, 1, 128, 64, 0, 8, 1), 3)]       # more than 8 query heads per kv head
    for (nh, nkv, hd, ms, pos0, n, mode), status in cases:
        with pytest.raises(HHError) as e:
            ctx.attention_prefill(z, z, z, nh, nkv, hd, ms, pos0, n, mode, z)
        assert e.value.status == status, (nh, nkv, hd, ms, pos0, n, mode, e.value)
