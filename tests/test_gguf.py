"""GGUF reader and model loader (hh_gguf_*, hh_model_load_gguf).

CPU tests parse files written by tests/gguf_writer.py through the C ABI (no
GPU call is made): header and alignment, every metadata type, the tensor table
and byte sizes, the error arms of GgufFile::open (gguf.rs:12-27, :138-218),
and ModelConfig::from_gguf (config.rs:57-217) with the qwen35 GDN geometry
(qwen35.rs:470-530).  The context cap is pinned to the known answers of the
reference's own kv_budget tests (kv_budget.rs:85-125).  The GPU test writes a
synthesized model to a GGUF file, loads it back and checks logits and tokens
are bit-identical.
"""
import os

import numpy as np
import pytest

from hearth_amd import GGML_Q2_0, GGML_Q8_0, HHError, lib as hl
import gguf_writer as gw

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def L():
    return hl.load_library()


def _rand_bytes(rng, t, shape):
    return rng.integers(0, 256, gw.tensor_nbytes(t, shape), dtype=np.uint8).tobytes()


def test_header_metadata_and_tensor_table(tmp_path, L):
    rng = np.random.default_rng(1)
    meta = [("general.architecture", gw.STRING, "qwen3"),
            ("k.u8", gw.U8, 200), ("k.i8", gw.I8, -5), ("k.u16", gw.U16, 60000), ("k.i16", gw.I16, -300),
            ("k.u32", gw.U32, 4000000000), ("k.i32", gw.I32, -7), ("k.f32", gw.F32, 0.15625),
            ("k.bool", gw.BOOL, 1), ("k.str", gw.STRING, "héllo"), ("k.u64", gw.U64, 1 << 40),
            ("k.i64", gw.I64, -(1 << 40)), ("k.f64", gw.F64, 2.5),
            ("k.arr", gw.ARRAY, (gw.STRING, ["a", "bb", "ccc"])),
            ("k.nested", gw.ARRAY, (gw.ARRAY, [(gw.U32, [1, 2]), (gw.U32, [3])]))]
    tensors = [("a.weight", 8, (64, 3), _rand_bytes(rng, 8, (64, 3))),
               ("b.weight", 42, (256, 2), _rand_bytes(rng, 42, (256, 2))),
               ("c.norm", 0, (7,), _rand_bytes(rng, 0, (7,))),
               ("d.q1", 41, (128, 5), _rand_bytes(rng, 41, (128, 5))),
               ("e.h", 1, (3, 3), _rand_bytes(rng, 1, (3, 3)))]
    p = str(tmp_path / "m.gguf")
    data_offset, offsets = gw.write_gguf(p, meta, tensors)
    with hl.Gguf(p, L) as g:
        v, off, al = g.header()
        assert (v, off, al) == (3, data_offset, 32) and off % 32 == 0
        info = g.tensors()
        assert [t["name"] for t in info] == [t[0] for t in tensors]
        for t, (name, ty, shape, data), o in zip(info, tensors, offsets):
            assert (t["type"], t["shape"], t["offset"], t["nbytes"]) == (ty, shape, o, len(data))
            assert g.tensor_bytes(info.index(t), t["nbytes"]) == data
        # MetaValue::as_u32 takes U32 and I32 (two's complement), nothing else
        assert g.meta_u32("k.u32") == 4000000000
        assert g.meta_u32("k.i32") == (1 << 32) - 7
        for k in ("k.u8", "k.u16", "k.u64", "k.f32", "k.str"):
            with pytest.raises(HHError):
                g.meta_u32(k)
        assert g.meta_f32("k.f32") == 0.15625
        with pytest.raises(HHError):
            g.meta_f32("k.f64")
        assert g.meta_str("k.str") == "héllo"
        assert g.meta_array_len("k.arr") == 3 and g.meta_array_len("k.nested") == 2
        with pytest.raises(HHError) as e:
            g.meta_u32("absent.key")
        assert e.value.status == hl.HH_ERR_NOT_FOUND


def test_v2_has_no_alignment_padding_and_custom_alignment(tmp_path, L):
    rng = np.random.default_rng(2)
    tensors = [("x", 8, (32, 1), _rand_bytes(rng, 8, (32, 1)))]
    p2 = str(tmp_path / "v2.gguf")
    d2, _ = gw.write_gguf(p2, [("general.architecture", gw.STRING, "llama")], tensors, version=2)
    with hl.Gguf(p2, L) as g:
        v, off, _ = g.header()
        assert v == 2 and off == d2
        assert g.tensor_bytes(0, 34) == tensors[0][3]
    p3 = str(tmp_path / "al.gguf")
    d3, _ = gw.write_gguf(p3, [("general.architecture", gw.STRING, "llama")], tensors, alignment=256)
    with hl.Gguf(p3, L) as g:
        v, off, al = g.header()
        assert (v, off, al) == (3, d3, 256) and off % 256 == 0
        assert g.tensor_bytes(0, 34) == tensors[0][3]


@pytest.mark.parametrize("case", ["magic", "version", "truncated_header", "truncated_meta", "unknown_dtype",
                                  "past_end", "missing"])
def test_open_errors(tmp_path, L, case):
    rng = np.random.default_rng(3)
    p = str(tmp_path / "bad.gguf")
    tensors = [("x", 8, (32, 2), _rand_bytes(rng, 8, (32, 2)))]
    meta = [("general.architecture", gw.STRING, "llama")]
    if case == "magic":
        gw.write_gguf(p, meta, tensors, magic=b"GGML")
    elif case == "version":
        gw.write_gguf(p, meta, tensors, version=4)
    elif case == "truncated_header":
        with open(p, "wb") as f:
            f.write(b"GGUF\x03\x00\x00\x00\x01")
    elif case == "truncated_meta":
        gw.write_gguf(p, meta, tensors)
        raw = open(p, "rb").read()
        open(p, "wb").write(raw[:40])
    elif case == "unknown_dtype":
        gw.write_gguf(p, meta, tensors)
        raw = bytearray(open(p, "rb").read())
        i = raw.index(b"x\x02\x00\x00\x00")        # name, n_dims = 2, then two u64 dims, then the type
        raw[i + 5 + 16:i + 5 + 20] = (77).to_bytes(4, "little")
        open(p, "wb").write(bytes(raw))
    elif case == "past_end":
        gw.write_gguf(p, meta, tensors)
        raw = open(p, "rb").read()
        open(p, "wb").write(raw[:-10])
    else:
        p = str(tmp_path / "does_not_exist.gguf")
    with pytest.raises(HHError) as e:
        hl.Gguf(p, L)
    want = {"unknown_dtype": hl.HH_ERR_DTYPE, "missing": hl.HH_ERR_NOT_FOUND}.get(case, hl.HH_ERR_INVALID)
    assert e.value.status == want, str(e.value)


def _config_file(tmp_path, cfg, name="c.gguf", arch=None, context_length=None, extra=(), drop=(),
                 explicit_hd=True, vocab_as_tokens=False):
    """A GGUF with the model's metadata and only the tensors config derivation reads."""
    rng = np.random.default_rng(4)
    meta = [m for m in gw.model_meta(cfg, arch=arch, context_length=context_length,
                                     vocab_as_tokens=vocab_as_tokens) if m[0].split(".", 1)[-1] not in drop]
    if not explicit_hd:
        meta = [m for m in meta if not m[0].endswith("attention.key_length")]
    meta += list(extra)
    hd, d = cfg.head_dim, 128
    tensors = [("token_embd.weight", cfg.head_type, (d, 4), None),
               ("blk.0.ffn_gate.weight", cfg.wtype, (d, 2), None)]
    if cfg.arch == 0:
        tensors.append(("blk.0.attn_q.weight", cfg.wtype, (d, cfg.n_heads * hd), None))
        if cfg.qk_norm:
            tensors.append(("blk.0.attn_q_norm.weight", 0, (hd,), None))
    else:
        a = cfg.full_attn_interval - 1
        tensors.append((f"blk.{a}.attn_k.weight", cfg.wtype, (d, cfg.n_kv_heads * hd), None))
        tensors.append((f"blk.{a}.attn_q_norm.weight", 0, (hd,), None))
    tensors = [(n, t, s, _rand_bytes(rng, t, s)) for n, t, s, _ in tensors]
    p = str(tmp_path / name)
    gw.write_gguf(p, meta, tensors)
    return p


def _derive(L, p, cap=0):
    with hl.Gguf(p, L) as g:
        return g.model_config(cap)


def test_config_dense_8b(tmp_path, L):
    cfg = hl.CONFIGS["8b-q2"].replace(max_seq=32768)
    c = _derive(L, _config_file(tmp_path, cfg, vocab_as_tokens=True))
    for f in ("arch", "d_model", "n_layers", "n_heads", "n_kv_heads", "head_dim", "d_ffn", "vocab", "wtype",
              "head_type", "qk_norm"):
        assert getattr(c, f) == getattr(cfg, f), f
    assert c.eps == np.float32(cfg.eps) and c.rope_theta == cfg.rope_theta and c.rope_dim == 128
    # kv_budget.rs:97-106: 36 x 8 x 128 (288 KiB per token) declaring 32768 -> 4096
    assert c.max_seq == 4096
    assert _derive(L, _config_file(tmp_path, cfg, name="o.gguf"), cap=2304).max_seq == 2304   # HEARTH_CTX_CAP
    assert _derive(L, _config_file(tmp_path, cfg.replace(max_seq=1000), name="s.gguf")).max_seq == 1000


def test_config_dense_1p7b_and_defaults(tmp_path, L):
    cfg = hl.CONFIGS["1.7b-q1"].replace(max_seq=32768)
    # kv_budget.rs:85-95: 28 x 8 x 128 declaring 32768 -> 4096
    assert _derive(L, _config_file(tmp_path, cfg)).max_seq == 4096
    # head_dim from attn_q rows when unstated (mod.rs:156-167); eps/theta/context defaults
    p = _config_file(tmp_path, cfg.replace(head_dim=96), name="d.gguf", explicit_hd=False,
                     drop=("rope.freq_base", "attention.layer_norm_rms_epsilon", "context_length",
                           "rope.dimension_count"))
    c = _derive(L, p)
    assert c.head_dim == 96 and c.rope_dim == 96
    assert c.eps == np.float32(1e-5) and c.rope_theta == 10000.0 and c.max_seq == 2048
    # llama.* fallback keys (config.rs:70-82) and the "llama" arch prefix
    c = _derive(L, _config_file(tmp_path, cfg, name="l.gguf", arch="llama"))
    assert (c.d_model, c.n_layers, c.arch) == (cfg.d_model, cfg.n_layers, 0)


def test_config_hybrid(tmp_path, L):
    cfg = hl.CONFIGS["27b-hybrid-pq2"].replace(max_seq=262144, rope_dim=64)
    c = _derive(L, _config_file(tmp_path, cfg))
    for f in ("arch", "d_model", "n_layers", "n_heads", "n_kv_heads", "head_dim", "d_ffn", "vocab", "wtype",
              "full_attn_interval", "ssm_n_k_heads", "ssm_n_v_heads", "ssm_head_dim", "ssm_conv_kernel",
              "attn_out_gate", "rope_dim"):
        assert getattr(c, f) == getattr(cfg, f), f
    # kv_budget.rs:108-122: 16 attention layers x 4 x 256 (128 KiB per token)
    # declaring 262144 -> 1.25 GiB / 128 KiB = 10240 (no dense 4096 cap)
    assert c.max_seq == 10240
    bad = _config_file(tmp_path, cfg, name="b.gguf", drop=("ssm.inner_size",),
                       extra=[("qwen35.ssm.inner_size", gw.U32, 1234)])
    with pytest.raises(HHError, match="inner_size"):
        _derive(L, bad)
    miss = _config_file(tmp_path, cfg, name="m.gguf", drop=("ssm.state_size",))
    with pytest.raises(HHError, match="state_size"):
        _derive(L, miss)


def test_config_absurd_kv_is_floored(tmp_path, L):
    # kv_budget.rs:124-129: 64 KV layers x 32 x 1024 (16 MiB per token) -> MIN_CTX 512
    cfg = hl.ModelConfig(d_model=1024, n_layers=64, n_heads=32, n_kv_heads=32, head_dim=1024, d_ffn=2048,
                         vocab=64, max_seq=1 << 20, wtype=GGML_Q2_0)
    assert _derive(L, _config_file(tmp_path, cfg)).max_seq == 512


def test_config_rejects_off_path_models(tmp_path, L):
    cfg = hl.CONFIGS["8b-q2"]
    with pytest.raises(HHError, match="architecture"):
        _derive(L, _config_file(tmp_path, cfg, name="g.gguf", arch="gemma2"))


def test_config_hadamard_fold(tmp_path, L):
    """prism.hadamard.* (qwen35.rs:532-620): a valid fold sets had_block and the
    latent/tied flags; each malformed variant fails with the reference's message."""
    h = hl.CONFIGS["9b-hybrid-q2"]
    rng = np.random.default_rng(1)
    signs = {4096: rng.choice([-1, 1], 4096), 12288: rng.choice([-1, 1], 12288)}
    ok = _config_file(tmp_path, h, name="h.gguf", extra=gw.hadamard_meta(1024, signs, version=2, latent=True))
    c = _derive(L, ok)
    assert c.had_block == 1024 and c.had_flags == 1
    plain = _derive(L, _config_file(tmp_path, h, name="p.gguf"))
    assert plain.had_block == 0 and plain.had_flags == 0
    bad = [
        (dict(version=3), "unsupported prism.hadamard.version 3"),
        (dict(transform="dct"), "unsupported hadamard transform dct"),
        (dict(signs={1000: np.ones(1000)}), "invalid hadamard sign width 1000"),
        (dict(signs={1024: np.full(1024, 2)}), "sign values must be"),
        (dict(tied=True, version=2), "requires a latent token_embd"),
        (dict(tied=True, version=1, latent=True), "requires prism.hadamard version 2"),
    ]
    for i, (kw, msg) in enumerate(bad):
        args = dict(signs=signs, version=1)
        args.update(kw)
        sg = args.pop("signs")
        p = _config_file(tmp_path, h, name=f"b{i}.gguf", extra=gw.hadamard_meta(1024, sg, **args))
        with pytest.raises(HHError, match=msg):
            _derive(L, p)
    # sign_values longer than the widths cover
    meta = gw.hadamard_meta(1024, signs)
    meta[4] = ("prism.hadamard.sign_values", gw.ARRAY, (gw.I8, list(meta[4][2][1]) + [1]))
    with pytest.raises(HHError, match="length mismatch"):
        _derive(L, _config_file(tmp_path, h, name="m.gguf", extra=meta))


def _write_model(m, path, tied=False, f16_norms=False):
    """Every tensor of a device model, as the GGUF a converter would write."""
    tensors = []
    for name, t, ne0, ne1, nb in m.tensors():
        if tied and name == "output.weight":
            continue
        data = m.download(name, nb).tobytes()
        shape = (ne0,) if ne1 == 1 and t == 0 else (ne0, ne1)
        if f16_norms and t == 0 and name.endswith("norm.weight"):
            data = np.frombuffer(data, np.float32).astype(np.float16).tobytes()
            t = 1
        tensors.append((name, t, shape, data))
    gw.write_gguf(path, gw.model_meta(m.cfg), tensors)


@pytest.mark.gpu
@pytest.mark.parametrize("which", ["dense", "hybrid", "dense_tied_f16"])
def test_load_gguf_matches_synthesized_model(tmp_path, ctx, which):
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import make_golden
    cfg = make_golden.HYBRID if which == "hybrid" else make_golden.DENSE
    ref = hl.Model(ctx, cfg)
    ref.synthesize(7)
    tied = f16 = which == "dense_tied_f16"
    if tied:   # the tied head reads token_embd; make the reference agree
        emb = ref.download("token_embd.weight", [t for t in ref.tensors() if t[0] == "token_embd.weight"][0][4])
        ref.upload("output.weight", GGML_Q8_0, cfg.d_model, cfg.vocab, emb)
    if f16:    # norms stored as F16 are widened; make the reference hold the same values
        for name, t, ne0, ne1, nb in ref.tensors():
            if t == 0 and name.endswith("norm.weight"):
                v = ref.download(name, nb).view(np.float32).astype(np.float16).astype(np.float32)
                ref.upload(name, 0, ne0, ne1, v)
    p = str(tmp_path / f"{which}.gguf")
    _write_model(ref, p, tied=tied, f16_norms=f16)
    m = hl.Model.from_gguf(ctx, p, ctx_cap=cfg.max_seq)
    for f in ("arch", "d_model", "n_layers", "n_heads", "n_kv_heads", "head_dim", "d_ffn", "vocab", "wtype",
              "head_type", "max_seq", "qk_norm", "attn_out_gate"):
        assert getattr(m.cfg, f) == getattr(cfg, f), f
    if cfg.arch == 1:
        for f in ("full_attn_interval", "ssm_n_k_heads", "ssm_n_v_heads", "ssm_head_dim", "ssm_conv_kernel",
                  "rope_dim"):
            assert getattr(m.cfg, f) == getattr(cfg, f), f
    for name, t, ne0, ne1, nb in ref.tensors():
        assert np.array_equal(m.download(name, nb), ref.download(name, nb)), name
    prompt = [11, 400, 7, 123]
    la, _ = ref.forward(prompt[0], 0)
    lb, _ = m.forward(prompt[0], 0)
    assert np.array_equal(la, lb)
    ref.reset()
    m.reset()
    ta, _ = ref.generate(prompt, 8, 0, 1.0)
    tb, _ = m.generate(prompt, 8, 0, 1.0)
    assert np.array_equal(ta, tb)
    m.close()
    ref.close()
