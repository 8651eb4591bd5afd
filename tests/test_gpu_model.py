"""GPU parity of whole decode steps and the token loop against the CPU oracle.

Bars (north star): synthesized weight bytes bit-exact; logits within 1e-3
relative (max |diff| / max |ref|); greedy tokens identical for the first 32.

The oracle runs in its device association order (the HIP kernels' reduction
grouping, same mathematics): GEMVs, quantization, norms, attention and the GDN
step then agree bit for bit, so the logits are compared for equality as well as
against the 1e-3 bar.  The reference-order oracle is compared at a looser bar
in test_reference_order_spread and tests/test_golden.py: there every reduction
regroups, which moves logits by Q8_0 rounding flips, as the reference's own
scalar and AVX2 GEMV arms do to each other."""
import numpy as np
import pytest

from hearth_amd.lib import ModelConfig, GGML_Q1_0, GGML_Q2_0, GGML_Q1_0_G128, GGML_PQ2_0, GGML_PTQ1_0, CONFIGS

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

TINY = ModelConfig(d_model=1024, n_layers=2, n_heads=8, n_kv_heads=4, head_dim=128, d_ffn=2048,
                   vocab=4096, max_seq=128, wtype=GGML_Q2_0)
TINY_HYB = ModelConfig(arch=1, d_model=1024, n_layers=4, n_heads=4, n_kv_heads=2, head_dim=256, rope_dim=64,
                       d_ffn=2048, vocab=4096, max_seq=128, wtype=GGML_Q2_0, full_attn_interval=4,
                       ssm_n_k_heads=2, ssm_n_v_heads=4, ssm_head_dim=128, ssm_conv_kernel=4,
                       attn_out_gate=1)


def rel(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / np.abs(b).max())


def make(ctx, oracle, cfg, seed, threads=16, order=1):
    from hearth_amd import Model
    m = Model(ctx, cfg)
    m.synthesize(seed)
    o = oracle.OracleModel(cfg, seed=seed, threads=threads, order=order)
    return m, o


@pytest.mark.parametrize("cfg", [TINY, TINY_HYB, TINY.replace(wtype=GGML_Q1_0), TINY_HYB.replace(wtype=GGML_PQ2_0),
                                 TINY.replace(wtype=GGML_PTQ1_0)],
                         ids=["dense-q2", "hybrid-q2", "dense-q1", "hybrid-pq2", "dense-ptq1"])
def test_synthesized_bytes_bit_exact(ctx, oracle, cfg):
    m, o = make(ctx, oracle, cfg, seed=21)
    names = o.tensor_names()
    dev = {t[0]: t for t in m.tensors()}
    assert sorted(names) == sorted(dev)
    for n in names:
        want = o.tensor(n)
        got = m.download(n, want.size)
        assert np.array_equal(got, want), n


@pytest.mark.parametrize("cfg", [TINY, TINY.replace(wtype=GGML_Q1_0), TINY_HYB, TINY.replace(wtype=GGML_PTQ1_0),
                                 TINY.replace(wtype=GGML_Q1_0_G128), TINY_HYB.replace(wtype=GGML_Q1_0)],
                         ids=["dense-q2", "dense-q1", "hybrid-q2", "dense-ptq1", "dense-q1g128", "hybrid-q1"])
def test_forward_logits_parity(ctx, oracle, cfg):
    m, o = make(ctx, oracle, cfg, seed=5)
    for pos, tok in enumerate([17, 400, 9, 4095, 0, 1234]):
        print(f"forward pos={pos}", flush=True)
        lg, am = m.forward(tok, pos)
        lw = o.forward(tok, pos)
        assert rel(lg, lw) < 1e-3, pos
        assert np.array_equal(lg, lw), (pos, rel(lg, lw))
        assert np.isfinite(lg).all()


@pytest.mark.parametrize("cfg,pen", [(TINY, 1.1), (TINY, 1.0), (TINY.replace(wtype=GGML_Q1_0), 1.1),
                                     (TINY_HYB, 1.0), (TINY_HYB.replace(wtype=GGML_PTQ1_0), 1.0)],
                         ids=["dense-pen", "dense", "dense-q1", "hybrid", "hybrid-ptq1"])
def test_generate_tokens_parity(ctx, oracle, cfg, pen):
    m, o = make(ctx, oracle, cfg, seed=7)
    prompt = [oracle.synth_token(7, i, cfg.vocab) for i in range(5)]
    toks, lg = m.generate(prompt, 32, repeat_pen=pen, want_logits=True)
    tw, lw = o.generate(prompt, 32, repeat_pen=pen, want_logits=True)
    assert list(toks) == list(tw)
    assert rel(lg, lw) < 1e-3
    assert np.array_equal(lg, lw)


@pytest.mark.parametrize("K", [2, 3, 6])
def test_hybrid_conv_kernel_lengths(ctx, oracle, K):
    """The GDN causal conv at lengths other than qwen35's 4 (the loader takes 2..8):
    the decode step's generic form (conv length read at run time) and the batched
    prefill's conv-window hand-off, with prompts longer and shorter than the
    window, then 16 greedy tokens: equal to the device-order oracle token for
    token and in the last logits."""
    cfg = TINY_HYB.replace(ssm_conv_kernel=K)
    m, o = make(ctx, oracle, cfg, seed=23)
    for n_prompt in (12, 2):
        prompt = [oracle.synth_token(23, 50 * n_prompt + i, cfg.vocab) for i in range(n_prompt)]
        m.reset()
        o.reset()
        toks, lg = m.generate(prompt, 16, repeat_pen=1.0, want_logits=True)
        tw, lw = o.generate(prompt, 16, repeat_pen=1.0, want_logits=True)
        assert list(toks) == list(tw), n_prompt
        assert np.array_equal(lg, lw), n_prompt


@pytest.mark.parametrize("cfg", [TINY, TINY_HYB], ids=["dense", "hybrid"])
def test_generate_lengths_across_graph_batches(ctx, oracle, cfg):
    """hh_model_generate runs the first decode step with the embedding kernel,
    then steps whose embedding the previous k_head_final wrote, eight per graph
    launch and the rest one at a time: lengths on both sides of those
    boundaries, back to back on one model, equal the oracle token for token."""
    m, o = make(ctx, oracle, cfg, seed=19)
    pen = 1.1 if cfg.arch == 0 else 1.0
    for n_gen in (1, 2, 8, 9, 17):
        prompt = [oracle.synth_token(19, n_gen * 7 + i, cfg.vocab) for i in range(3)]
        m.reset()
        o.reset()
        toks, lg = m.generate(prompt, n_gen, repeat_pen=pen, want_logits=True)
        tw, lw = o.generate(prompt, n_gen, repeat_pen=pen, want_logits=True)
        assert list(toks) == list(tw), n_gen
        assert np.array_equal(lg, lw), n_gen
        m.reset()
        t2 = m.generate(prompt, n_gen, repeat_pen=pen)[0]   # no last logits: one step fewer
        assert list(t2) == list(tw), n_gen


def test_8b_shaped_prefilled_kv(ctx, oracle):
    """Config 3 geometry (d 4096, 32/8 heads, ffn 12288, vocab 151936) with 2
    layers, KV pre-filled to 2048 positions of seeded N(0,1) fp16 values, then
    greedy decode from pos 2048: logits and tokens against the oracle."""
    cfg = CONFIGS["8b-q2"].replace(n_layers=2)
    m, o = make(ctx, oracle, cfg, seed=3)
    m.prefill_kv_synthetic(99, 2048)
    o.prefill_kv_synthetic(99, 2048)
    tok0 = oracle.synth_token(3, 0, cfg.vocab)
    toks, lg = m.generate([tok0], 32, start_pos=2048, repeat_pen=1.1, want_logits=True)
    tw, lw = o.generate([tok0], 32, start_pos=2048, repeat_pen=1.1, want_logits=True)
    assert list(toks) == list(tw)
    assert rel(lg, lw) < 1e-3
    assert np.array_equal(lg, lw)


def test_8b_full_depth_bit_exact(ctx, oracle):
    """The benchmarked model itself: all 36 layers of the 8B Q2_0 geometry, KV
    pre-filled to 2048, four greedy steps with the 1.1 penalty through
    hh_model_generate (graph batches and the head's embedding hand-off
    included): tokens and the last logits equal the device-order oracle, which
    holds the same weights (downloaded from the device)."""
    cfg = CONFIGS["8b-q2"].replace(max_seq=2112)
    from hearth_amd import Model
    m = Model(ctx, cfg)
    m.synthesize(2026)
    o = oracle.OracleModel(cfg, seed=None, threads=16, order=oracle.OracleModel.DEVICE)
    for name, t, ne0, ne1, nb in m.tensors():
        o.tensor(name)[:] = m.download(name, nb)
    m.prefill_kv_synthetic(77, 2048)
    o.prefill_kv_synthetic(77, 2048)
    print("8b full depth: generating", flush=True)
    toks, lg = m.generate([5], 4, start_pos=2048, repeat_pen=1.1, want_logits=True)
    tw, lw = o.generate([5], 4, start_pos=2048, repeat_pen=1.1, want_logits=True)
    assert list(toks) == list(tw)
    assert np.array_equal(lg, lw)
    o.close()
    m.close()


@pytest.mark.parametrize("name", ["9b-hybrid-q2", "27b-hybrid-pq2"])
def test_hybrid_full_depth_bit_exact(ctx, oracle, name):
    """The benchmarked hybrids at full depth (9B: 32 layers; 27B PQ2_0: 64
    layers, d 5120, vocab 248320): a 12-token prompt through the batched
    prefill (MFMA GEMMs, GDN rows kernels, gated attention), then four greedy
    steps; tokens and the last logits equal the device-order oracle fed token
    by token on the same (downloaded) weights."""
    cfg = CONFIGS[name].replace(max_seq=64)
    from hearth_amd import Model
    m = Model(ctx, cfg)
    m.synthesize(31)
    o = oracle.OracleModel(cfg, seed=None, threads=16, order=oracle.OracleModel.DEVICE)
    for tname, t, ne0, ne1, nb in m.tensors():
        o.tensor(tname)[:] = m.download(tname, nb)
    prompt = [oracle.synth_token(31, i, cfg.vocab) for i in range(12)]
    print(f"{name} full depth: generating", flush=True)
    toks, lg = m.generate(prompt, 4, want_logits=True)
    tw, lw = o.generate(prompt, 4, want_logits=True)
    assert list(toks) == list(tw)
    assert np.array_equal(lg, lw)
    o.close()
    m.close()


@pytest.mark.parametrize("cfg,kv_type", [(CONFIGS["8b-q2"].replace(n_layers=1, max_seq=8192), 0),
                                         (CONFIGS["8b-q2"].replace(n_layers=1, max_seq=8192), 8),
                                         (CONFIGS["9b-hybrid-q2"].replace(n_layers=4, max_seq=8192), 0)],
                         ids=["8b-f32", "8b-kvq8", "9b-hybrid"])
def test_long_context_decode(ctx, oracle, cfg, kv_type):
    """Decode at 7936 prefilled positions: 124 attention chunks per kv head at
    head_dim 128 (248 at 256), so the merge walks more partials than a wave
    has lanes.  Logits and tokens equal the device-order oracle."""
    cfg = cfg.replace(kv_type=kv_type)
    m, o = make(ctx, oracle, cfg, seed=4)
    m.prefill_kv_synthetic(41, 7936)
    o.prefill_kv_synthetic(41, 7936)
    tok0 = oracle.synth_token(4, 0, cfg.vocab)
    pen = 1.1 if cfg.arch == 0 else 1.0
    toks, lg = m.generate([tok0], 8, start_pos=7936, repeat_pen=pen, want_logits=True)
    tw, lw = o.generate([tok0], 8, start_pos=7936, repeat_pen=pen, want_logits=True)
    assert list(toks) == list(tw)
    assert np.array_equal(lg, lw)
    o.close()


@pytest.mark.parametrize("seed", [9, 10, 11])
@pytest.mark.parametrize("cfg", [TINY, TINY_HYB], ids=["dense", "hybrid"])
def test_reference_order_spread(ctx, oracle, cfg, seed):
    """Against the reference-order oracle over 8 decode steps: the device's
    logits are as close to the reference's scalar arm as the reference's own
    AVX2 arm is.  Every regrouped fp32 sum can flip a Q8_0 rounding of a later
    activation, so neither the AVX2 arm nor the device holds 1e-3 on whole-model
    logits once such a flip occurs; the bar is max(1e-3, 1.25 x the AVX2 arm's
    largest relative deviation over the same 8 steps)."""
    from hearth_amd import Model
    m = Model(ctx, cfg)
    m.synthesize(seed)
    ref = oracle.OracleModel(cfg, seed=seed, threads=16, arm=0, order=0)
    avx = oracle.OracleModel(cfg, seed=seed, threads=16, arm=1, order=0)
    arms, dev = [], []
    for pos, t in enumerate([123, 5, 900, 17, 3000, 44, 1, 2]):
        lr = ref.forward(t, pos)
        arms.append(rel(avx.forward(t, pos), lr))
        dev.append(rel(m.forward(t, pos)[0], lr))
    print(f"seed {seed}: AVX2 arm {np.round(arms, 4)}, device {np.round(dev, 4)}", flush=True)
    assert max(dev) <= max(1e-3, 1.25 * max(arms)), (dev, arms)
    m.close()


def test_model_errors(ctx):
    from hearth_amd import Model, HHError
    m = Model(ctx, TINY)
    with pytest.raises(HHError) as e:
        m.forward(1, TINY.max_seq)
    assert e.value.status == 7
    with pytest.raises(HHError) as e:
        m.forward(TINY.vocab, 0)
    assert e.value.status == 7
    with pytest.raises(HHError) as e:
        m.generate([], 3)
    assert e.value.status == 1
    m.set_cancel(True)
    with pytest.raises(HHError) as e:
        m.forward(1, 0)
    assert e.value.status == 8
    m.set_cancel(False)
    m.forward(1, 0)
    with pytest.raises(HHError) as e:
        m.upload("blk.0.attn_q.weight", GGML_Q1_0, 1024, 1024, np.zeros(10, np.uint8))
    assert e.value.status == 2
    with pytest.raises(HHError) as e:
        m.upload("blk.99.attn_q.weight", GGML_Q2_0, 1024, 1024, np.zeros(10, np.uint8))
    assert e.value.status == 6
    with pytest.raises(HHError):
        Model(ctx, TINY.replace(d_model=1000))


def test_upload_roundtrip(ctx, oracle):
    """Weights uploaded from host bytes (the GGUF path) behave like synthesized ones."""
    from hearth_amd import Model
    cfg = TINY
    o = oracle.OracleModel(cfg, seed=13, threads=8)
    m = Model(ctx, cfg)
    for name, t, ne0, ne1, nb in m.tensors():
        m.upload(name, t, ne0, ne1, o.tensor(name))
    lg, _ = m.forward(5, 0)
    assert rel(lg, o.forward(5, 0)) < 1e-3


def _model_with_env(ctx, cfg, seed, env):
    import os
    from hearth_amd import Model
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        m = Model(ctx, cfg)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    m.synthesize(seed)
    return m


@pytest.mark.parametrize("cfg,n_prompt", [(TINY, 9), (TINY.replace(wtype=GGML_Q1_0), 40),
                                          (CONFIGS["8b-q2"].replace(n_layers=2, max_seq=640), 300),
                                          (TINY.replace(wtype=GGML_PTQ1_0), 33),
                                          (TINY_HYB, 3), (TINY_HYB, 9), (TINY_HYB.replace(wtype=GGML_PQ2_0), 37),
                                          (CONFIGS["9b-hybrid-q2"].replace(n_layers=4, max_seq=640), 300),
                                          (TINY.replace(kv_type=8), 9), (TINY_HYB.replace(kv_type=8), 9),
                                          (CONFIGS["8b-q2"].replace(n_layers=2, max_seq=640, kv_type=8), 300),
                                          (TINY.replace(n_heads=16, n_kv_heads=2, max_seq=160), 70),
                                          (TINY.replace(n_heads=12, n_kv_heads=4, max_seq=160), 70),
                                          (TINY.replace(n_heads=4, n_kv_heads=4, max_seq=160), 70),
                                          (TINY.replace(n_heads=32, n_kv_heads=32, max_seq=640), 600),
                                          (TINY.replace(n_heads=32, n_kv_heads=32, max_seq=640, kv_type=8), 600),
                                          (TINY.replace(head_dim=256, n_heads=16, n_kv_heads=16, max_seq=640), 600)],
                         ids=["dense-q2", "dense-q1", "8b-2layer-300", "dense-ptq1", "hybrid-2", "hybrid-8",
                              "hybrid-pq2-36", "9b-4layer-300", "dense-kvq8", "hybrid-kvq8", "8b-kvq8-300",
                              "dense-g8-70", "dense-g3-70", "dense-g1-70", "wide-chunks-600", "wide-chunks-kvq8-600",
                              "wide-chunks-hd256-600"])
def test_batched_prefill_equals_token_by_token(ctx, oracle, cfg, n_prompt):
    """forward_batch on the MFMA GEMM leaves the same KV cache (and, on the
    hybrids, the same conv windows and GDN states) as feeding the prompt one
    token at a time: the first generated token's logits and the next tokens are
    identical, and match the device-order oracle (at 300 tokens too: the
    oracle skips the LM head for prompt tokens).  hybrid-2 prefills fewer
    tokens than the conv window holds; the kvq8 cases write a Q8_0 cache
    (quantized on write as the decode step does); the g8 / g3 / g1 cases take
    the attention kernels' other query-group sizes (8 and 1 exact, 3 read at
    run time) over more than one 64-position chunk.  The wide-chunks cases have
    32 kv heads (16 at head_dim 256), so past 512 positions the attention
    splits take twice the positions per workgroup: the prompt's later tokens
    and the decode steps after it run the wide arithmetic."""
    print(f"prefill {cfg.d_model} {cfg.n_layers} n={n_prompt}", flush=True)
    pen = 1.1 if cfg.arch == 0 else 1.0
    prompt = [oracle.synth_token(11, i, cfg.vocab) for i in range(n_prompt)]
    mb = _model_with_env(ctx, cfg, 13, {"HH_BATCHED_PREFILL": "1"})
    mt = _model_with_env(ctx, cfg, 13, {"HH_BATCHED_PREFILL": "0"})
    tb, lb = mb.generate(prompt, 8, repeat_pen=pen, want_logits=True)
    tt, lt = mt.generate(prompt, 8, repeat_pen=pen, want_logits=True)
    assert list(tb) == list(tt)
    assert np.array_equal(lb, lt)
    o = oracle.OracleModel(cfg, seed=13, threads=16, order=oracle.OracleModel.DEVICE)
    tw, lw = o.generate(prompt, 8, repeat_pen=pen, want_logits=True)
    assert list(tb) == list(tw)
    assert np.array_equal(lb, lw)
    o.close()
    mb.close()
    mt.close()


@pytest.mark.parametrize("cfg", [TINY, TINY_HYB], ids=["dense", "hybrid"])
def test_prefill_then_forward(ctx, cfg):
    """hh_model_prefill(prompt[:-1]) in two calls (the second continues from the
    first's cache, conv windows and states) then hh_model_forward(last token)
    equals feeding every token through the decode step."""
    prompt = [5, 77, 1023, 4000, 12, 9, 300, 2, 4001, 18, 19]
    m = _model_with_env(ctx, cfg, 4, {"HH_BATCHED_PREFILL": "1"})
    m.prefill(prompt[:2], 0)
    m.prefill(prompt[2:-1], 2)
    lg, am = m.forward(prompt[-1], len(prompt) - 1)
    m2 = _model_with_env(ctx, cfg, 4, {"HH_BATCHED_PREFILL": "0"})
    for p, t in enumerate(prompt[:-1]):
        m2.forward(t, p)
    lg2, am2 = m2.forward(prompt[-1], len(prompt) - 1)
    assert np.array_equal(lg, lg2) and am == am2
    assert m.last_prefill_ms() > 0
    m.close()
    m2.close()


@pytest.mark.parametrize("cfg", [TINY, TINY_HYB], ids=["dense", "hybrid"])
def test_ptq1_0_model_equals_q2_0_model(ctx, cfg):
    """The generator gives a PTQ1_0 model the Q2_0 model's ternary weights: the
    two formats' decoders must then produce identical logits and tokens."""
    from hearth_amd import Model
    ma, mb = Model(ctx, cfg), Model(ctx, cfg.replace(wtype=GGML_PTQ1_0))
    ma.synthesize(31)
    mb.synthesize(31)
    prompt = [5, 900, 17, 3000]
    ta, la = ma.generate(prompt, 16, repeat_pen=1.1 if cfg.arch == 0 else 1.0, want_logits=True)
    tb, lb = mb.generate(prompt, 16, repeat_pen=1.1 if cfg.arch == 0 else 1.0, want_logits=True)
    assert list(ta) == list(tb)
    assert np.array_equal(la, lb)
    ma.close()
    mb.close()


@pytest.mark.parametrize("cfg,pen", [(TINY.replace(kv_type=8), 1.1), (TINY_HYB.replace(kv_type=8), 1.0)],
                         ids=["dense", "hybrid"])
def test_q8_0_kv_cache_parity(ctx, oracle, cfg, pen):
    """KVStorage::Q8_0 (kvcache.rs:41-57): rows quantized on write, attention over
    the dequantized rows (attention_q8_0, ops.rs:946-1030).  Logits and tokens
    equal the device-order oracle holding dequant(quantize(row))."""
    m, o = make(ctx, oracle, cfg, seed=17)
    prompt = [oracle.synth_token(17, i, cfg.vocab) for i in range(6)]
    toks, lg = m.generate(prompt, 24, repeat_pen=pen, want_logits=True)
    tw, lw = o.generate(prompt, 24, repeat_pen=pen, want_logits=True)
    assert list(toks) == list(tw)
    assert rel(lg, lw) < 1e-3
    assert np.array_equal(lg, lw)
    # the cache is really quantized: the f32-cache model diverges from it
    o32 = oracle.OracleModel(cfg.replace(kv_type=0), seed=17, threads=16, order=1)
    _, l32 = o32.generate(prompt, 24, repeat_pen=pen, want_logits=True)
    assert not np.array_equal(lg, l32)
    o32.close()


def test_q8_0_kv_prefilled_8b_shape(ctx, oracle):
    """8B geometry, 2 layers, Q8_0 KV prefilled to 2048 positions (the seeded
    fp16 values quantized per 32-block), greedy decode from pos 2048."""
    cfg = CONFIGS["8b-q2"].replace(n_layers=2, kv_type=8)
    m, o = make(ctx, oracle, cfg, seed=3)
    m.prefill_kv_synthetic(99, 2048)
    o.prefill_kv_synthetic(99, 2048)
    tok0 = oracle.synth_token(3, 0, cfg.vocab)
    toks, lg = m.generate([tok0], 16, start_pos=2048, repeat_pen=1.1, want_logits=True)
    tw, lw = o.generate([tok0], 16, start_pos=2048, repeat_pen=1.1, want_logits=True)
    assert list(toks) == list(tw)
    assert np.array_equal(lg, lw)


