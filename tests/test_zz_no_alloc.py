"""hh_attention_noalloc (the allocation-free variant of hh_attention, its split
partials in the library's fixed per-GPU scratch) against hh_attention through
the C ABI: bit-identical outputs on two calls in a row, the second smaller and
of another geometry, and a clear error for a call beyond the scratch."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _case(ctx, rng, nh, nkv, hd, ms, seq):
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    q = dev(rng.standard_normal(nh * hd).astype(np.float32))
    k = dev(rng.standard_normal(nkv * ms * hd).astype(np.float32))
    v = dev(rng.standard_normal(nkv * ms * hd).astype(np.float32))
    a = torch.zeros(nh * hd, dtype=torch.float32, device="cuda")
    b = torch.full((nh * hd,), float("nan"), dtype=torch.float32, device="cuda")
    ctx.attention(q, k, v, nh, nkv, hd, ms, seq, a)
    ctx.attention_noalloc(q, k, v, nh, nkv, hd, ms, seq, b)
    ctx.sync()
    return a.cpu().numpy(), b.cpu().numpy()


def test_noalloc_attention_equals_hh_attention(ctx):
    rng = np.random.default_rng(12)
    print("noalloc: 32/8 x 128, seq 2049", flush=True)
    a, b = _case(ctx, rng, 32, 8, 128, 2304, 2049)
    assert np.isfinite(a).all() and np.array_equal(a, b)
    print("noalloc: 16/4 x 256, seq 300", flush=True)
    a, b = _case(ctx, rng, 16, 4, 256, 512, 300)
    assert np.isfinite(a).all() and np.array_equal(a, b)


def test_noalloc_attention_rejects_beyond_scratch(ctx):
    from hearth_amd import HHError
    nh, nkv, hd, ms = 32, 8, 128, 40000
    q = torch.zeros(nh * hd, dtype=torch.float32, device="cuda")
    kv = torch.zeros(nkv * ms * hd, dtype=torch.float32, device="cuda")
    out = torch.zeros(nh * hd, dtype=torch.float32, device="cuda")
    with pytest.raises(HHError) as e:   # 8 x 625 splits x 4 x 130 floats > 4 MiB
        ctx.attention_noalloc(q, kv, kv, nh, nkv, hd, ms, 40000, out)
    assert e.value.status == 7 and "4 MiB" in str(e.value)


def test_attention_rejects_more_than_8_heads_per_kv_head(ctx):
    """G = n_heads / n_kv above 8 is a dimension error from both entry points."""
    from hearth_amd import HHError
    nh, nkv, hd, ms = 16, 1, 128, 64
    q = torch.zeros(nh * hd, dtype=torch.float32, device="cuda")
    kv = torch.zeros(nkv * ms * hd, dtype=torch.float32, device="cuda")
    out = torch.zeros(nh * hd, dtype=torch.float32, device="cuda")
    for call in (ctx.attention, ctx.attention_noalloc):
        with pytest.raises(HHError) as e:
            call(q, kv, kv, nh, nkv, hd, ms, 10, out)
        assert e.value.status == 3 and "8 query heads" in str(e.value)
