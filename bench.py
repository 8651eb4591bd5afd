"""Benchmark: batch-1 greedy decode of the 8B-shaped Q2_0 model at 2k context.

Workload (the north-star config): d_model 4096, 36
layers, 32 q / 8 kv heads x 128, SwiGLU 12288, vocab 151936; Q2_0 layer weights
and Q8_0 embedding/head synthesized on the device from a seed; f32 KV cache
pre-filled at positions 0..2047 with seeded N(0,1) values rounded to fp16; then
greedy decode (repetition penalty 1.1, the reference default) from position 2048.
A "step" is one decode forward (one token).  Timed region: K steps on the device
stream, bracketed by synchronize + hipEvents inside the library.

Also reported: per-stage device times (hipEvents) for layer 0, the roofline of
the dominant kernel (the fused gate/up Q2_0 GEMV), and the CPU baseline — the
oracle's restatement of Hearth's CPU path (AVX2 LUT Q2_0 arm, pool.rs row
partitioning) timed on the host's cores on a bounded sample of the same work.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
# HBM bytes per launch come from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
# summary (scaled by a plain copy's counts), read at run time.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_8b_q2_hbm_traffic.txt")
METRIC = "decode tok/s @bs1, 8B Q2_0 2k ctx; Q1/Q2 GEMV HBM GB/s vs peak"


def step_bytes(cfg, seq_len: int) -> dict:
    """Algorithmic HBM bytes of one decode step at attention length seq_len."""
    from hearth_amd import row_bytes
    d, L, hd = cfg.d_model, cfg.n_layers, cfg.head_dim
    nq, nkv = cfg.n_heads * hd, cfg.n_kv_heads * hd
    rb = lambda k: row_bytes(cfg.wtype, k)
    w_layer = (nq + 2 * nkv) * rb(d) + d * rb(nq) + 2 * cfg.d_ffn * rb(d) + d * rb(cfg.d_ffn)
    head = cfg.vocab * row_bytes(cfg.head_type, d)
    row = hd + hd // 32 * 2 if cfg.kv_type == 8 else hd * 4   # Q8_0 row: int8 + f16 block scales
    kv_read = L * 2 * cfg.n_kv_heads * seq_len * row
    kv_write = L * 2 * cfg.n_kv_heads * row
    norms = L * (2 * d + 2 * hd) * 4 + d * 4
    small = row_bytes(cfg.head_type, d) + cfg.vocab * 4
    return {"weights": L * w_layer, "head": head, "kv": kv_read + kv_write, "other": norms + small,
            "total": L * w_layer + head + kv_read + kv_write + norms + small,
            "gate_up": 2 * cfg.d_ffn * rb(d) + d * 4 * 2 + cfg.d_ffn + cfg.d_ffn // 32 * 8,
            # attn_output and ffn_down: weights, packed activation in, y read + written
            "out_proj": d * rb(nq) + nq + nq // 32 * 8 + d * 8,
            "down": d * rb(cfg.d_ffn) + cfg.d_ffn + cfg.d_ffn // 32 * 8 + d * 8,
            "in_proj": (nq + 2 * nkv) * rb(d) + d * 4 * 2 + (nq + 2 * nkv) * 4,
            # one layer's attention: K and V rows read, the new row written
            "attention": 2 * cfg.n_kv_heads * seq_len * row + 2 * cfg.n_kv_heads * row}


GEMV_SOURCE = os.path.join(ROOT, "hearth_amd", "csrc", "hh_gemv.hip")


def gemv_source_hash() -> str:
    import hashlib
    with open(GEMV_SOURCE, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def traffic_is_current() -> bool:
    """The counter summary records the hash of hh_gemv.hip it was measured on;
    a summary of other GEMV code is stale."""
    try:
        with open(TRAFFIC_FILE) as f:
            for ln in f:
                if ln.startswith("GEMV source (hh_gemv.hip) sha256:"):
                    return ln.split(":", 1)[1].strip() == gemv_source_hash()
    except OSError:
        pass
    return False


def measured_traffic(kernel_prefix: str):
    """HBM bytes per dispatch of a kernel from the committed counter summary
    (the 'traffic MB' column); None when the summary has no such row or was
    measured on another version of the GEMV source."""
    if not traffic_is_current():
        return None
    try:
        with open(TRAFFIC_FILE) as f:
            for ln in f:
                if ln.startswith(kernel_prefix):
                    cols = ln[len(kernel_prefix):].split()
                    return int(float(cols[-3]) * 1e6)
    except (OSError, ValueError, IndexError):
        pass
    return None


def cpu_baseline(model, cfg, seed, kv_seed, tok0, budget_s: float):
    """The oracle's restatement of Hearth's CPU decode, same weights (downloaded),
    T = host cores, AVX2 arm; decode steps until ~budget_s of CPU work."""
    from oracle import oracle as orc
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = max(1, min(threads, 16))
    o = orc.OracleModel(cfg, seed=None, threads=threads, arm=1)
    for name, t, ne0, ne1, nb in model.tensors():
        o.tensor(name)[:] = model.download(name, nb)
    o.prefill_kv_synthetic(kv_seed, 2048)
    tok, pos, n = tok0, 2048, 0
    t0 = time.perf_counter()
    while True:
        lg = o.forward(tok, pos)
        tok = int(np.argmax(lg))
        pos += 1
        n += 1
        el = time.perf_counter() - t0
        if el > budget_s or n >= 64:
            break
    o.close()
    avx2 = bool(orc.load().ho_have_avx2())
    host = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            host = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), host)
    except OSError:
        pass
    return {"value": n / el, "unit": "tok/s", "cores": threads, "kind": "port",
            "host_cpu": host, "nproc": os.cpu_count(),
            "sample": f"{n} decode steps of the 8B Q2_0 config from pos 2048 (f32 KV), "
                      f"{'AVX2 LUT' if avx2 else 'scalar'} Q2_0 arm, {threads} threads, {el:.1f} s"}


PEAK_INT8_TOPS = 5000.0


def prefill_leg(m, cfg, n_tok: int) -> dict:
    """forward_batch of an n_tok seeded prompt at positions 0.. (overwrites the
    synthetic KV; runs after the decode measurement).  The layer GEMMs run on
    int8 MFMA; attention and the row kernels on the vector units."""
    rng = np.random.default_rng(7)
    toks = rng.integers(0, cfg.vocab, n_tok).tolist()
    m.prefill(toks[:64], 0)                       # warm-up (scratch, code)
    m.prefill(toks, 0)
    ms = m.last_prefill_ms()
    d, hd = cfg.d_model, cfg.head_dim
    n_in = (cfg.n_heads + 2 * cfg.n_kv_heads) * hd
    weights = cfg.n_layers * (n_in * d + d * cfg.n_heads * hd + 2 * cfg.d_ffn * d + d * cfg.d_ffn)
    gemm_ops = 2.0 * n_tok * weights
    tops = gemm_ops / (ms * 1e-3) / 1e12
    print(f"[bench] prefill {n_tok} tokens: {ms:.2f} ms ({n_tok / (ms * 1e-3):.0f} tok/s)", file=sys.stderr, flush=True)
    return {"tokens": n_tok, "ms": round(ms, 3), "tok_per_s": round(n_tok / (ms * 1e-3), 1),
            "gemm_int8_ops": gemm_ops, "int8_TOPS_over_whole_prefill": round(tops, 1),
            "mfma_frac": round(tops / PEAK_INT8_TOPS, 4), "peak_int8_TOPS": PEAK_INT8_TOPS,
            "note": "int8 ops of the layer GEMMs only, divided by the whole prefill time (attention and row "
                    "kernels included); dense-model forward_batch, bit-identical to token-by-token decode"}


def prefill_mfma_attention_leg(ctx, cfg, seed: int, n_tok: int) -> dict:
    """The same 2048-token prefill with its attention on fp32 MFMA
    (HH_PREFILL_ATTN=mfma, k_attn_prefill_mfma): fp32-rounding parity with the
    default split/merge attention instead of bit parity with decode."""
    from hearth_amd import Model
    os.environ["HH_PREFILL_ATTN"] = "mfma"
    try:
        m = Model(ctx, cfg)
    finally:
        os.environ.pop("HH_PREFILL_ATTN", None)
    m.synthesize(seed)
    r = prefill_leg(m, cfg, n_tok)
    m.close()
    r["note"] = ("opt-in HH_PREFILL_ATTN=mfma: causal attention on fp32 MFMA (flash form, online softmax); "
                 "within 1e-5 of float64 attention, logits within fp32-rounding/Q8_0-flip distance of the default")
    return r


def kv_q8_leg(ctx, cfg, seed, kv_seed, tok0, K, W) -> dict:
    """The same decode with the KV cache held as Q8_0 rows (KVStorage::Q8_0,
    kvcache.rs:41-57): 3.8x fewer KV bytes at 2k context.  Reported beside the
    headline, which keeps the reference's default f32 cache."""
    from hearth_amd import Model
    c8 = cfg.replace(kv_type=8)
    m = Model(ctx, c8)
    m.synthesize(seed)
    m.prefill_kv_synthetic(kv_seed, 2048)
    if W:
        m.generate([tok0], W + 1, start_pos=2048, repeat_pen=1.1)
    m.generate([tok0], K + 1, start_pos=2048, repeat_pen=1.1)
    ms = m.last_decode_ms() / K
    stage = m.time_stages(layer=0, iters=50)
    m.close()
    b = step_bytes(c8, int(round(2048 + 1 + (K - 1) / 2.0 + 1)))
    tps = 1000.0 / ms
    print(f"[bench] Q8_0 KV: {ms:.4f} ms/step ({tps:.1f} tok/s), mix {stage['mix'] * 1e3:.2f} us",
          file=sys.stderr, flush=True)
    return {"tok_per_s": round(tps, 2), "ms_per_step": round(ms, 4), "bytes_per_step": b["total"],
            "step_hbm_frac": round(b["total"] * tps / 1e9 / PEAK_HBM_GBS, 4),
            "attention_stage_ms": round(stage["mix"], 5),
            "note": "same model and prompt with a Q8_0 KV cache (an option of the reference, not its default)"}


def _generate_leg(ctx, name: str, cfg, seed: int, n_prompt: int, n_gen: int, pen: float) -> dict:
    """Seeded prompt through generate (batched prefill of all prompt tokens but
    the last, then the decode graph); prefill and decode timed separately on
    the device."""
    from hearth_amd import Model
    m = Model(ctx, cfg)
    m.synthesize(seed)
    rng = np.random.default_rng(seed)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab, n_prompt)]
    m.generate(prompt[:16], 2, repeat_pen=pen)          # warm-up (scratch, code)
    m.reset()
    toks, _ = m.generate(prompt, n_gen, repeat_pen=pen)
    pf_ms = m.last_prefill_ms()
    dec_ms = m.last_decode_ms() / max(1, n_gen - 1)
    m.close()
    print(f"[bench] {name}: prompt {n_prompt} tokens {pf_ms:.1f} ms ({n_prompt / (pf_ms * 1e-3):.0f} tok/s), "
          f"decode {dec_ms:.4f} ms/step ({1000.0 / dec_ms:.1f} tok/s)", file=sys.stderr, flush=True)
    return {"prompt_tokens": n_prompt, "prompt_ms": round(pf_ms, 2),
            "prompt_tok_per_s": round(n_prompt / (pf_ms * 1e-3), 1), "decode_steps": n_gen - 1,
            "decode_tok_per_s": round(1000.0 / dec_ms, 2), "decode_ms_per_step": round(dec_ms, 4),
            "repeat_pen": pen, "first_tokens": [int(t) for t in toks[:8]]}


def single_leg(ctx, name: str) -> dict:
    """One configs leg with the same workload as config_legs (for rocprofv3 runs)."""
    from hearth_amd import CONFIGS
    if name == "1.7b":
        c0 = CONFIGS["1.7b-q1"]
        return _generate_leg(ctx, "1.7B Q1_0", c0.replace(max_seq=max(c0.max_seq, 128)), 2025, 16, 50, 1.1)
    if name == "9b":
        c3 = CONFIGS["9b-hybrid-q2"]
        return _generate_leg(ctx, "9B hybrid Q2_0", c3.replace(max_seq=max(c3.max_seq, 1024)), 2027, 512, 129, 1.0)
    if name == "27b-decode":
        return _generate_leg(ctx, "27B hybrid PQ2_0 (decode)", CONFIGS["27b-hybrid-pq2"].replace(max_seq=8192), 2028,
                             64, 17, 1.0)
    return _generate_leg(ctx, "27B hybrid PQ2_0", CONFIGS["27b-hybrid-pq2"].replace(max_seq=8192), 2028, 2048, 65,
                         1.0)


def config_legs(ctx) -> dict:
    """BASELINE configs[0], [1], [3], [4] on the device (seeded synthetic weights).
    The prompt phase includes the last prompt token's decode step."""
    from hearth_amd import CONFIGS, microbench
    out = {}
    c0 = CONFIGS["1.7b-q1"]
    out["cfg0_1.7b_q1"] = _generate_leg(ctx, "1.7B Q1_0", c0.replace(max_seq=max(c0.max_seq, 128)), 2025, 16,
                                        50, 1.1)
    out["cfg0_1.7b_q1"]["workload"] = "1.7B-shaped Q1_0 dense, 16-token prompt, 50 greedy tokens"
    out["hbm_copy"] = microbench.copy_bandwidth()
    print(f"[bench] HBM copy {out['hbm_copy']['MiB']} MiB: {out['hbm_copy']['GB/s']} GB/s (read + write)",
          file=sys.stderr, flush=True)
    out["hbm_read"] = microbench.read_bandwidth()
    print(f"[bench] HBM read-only {out['hbm_read']['MiB']} MiB: {out['hbm_read']['GB/s']} GB/s",
          file=sys.stderr, flush=True)
    g = microbench.run(reps=1000, formats=("Q1_0", "Q2_0"), shapes=microbench.SHAPES[:3])
    out["cfg1_gemv"] = [{k: r[k] for k in ("format", "n", "k", "us", "GB/s", "frac_peak", "cache_resident_us",
                                           "cache_resident_GB/s")} for r in g]
    for r in g:
        print(f"[bench] GEMV {r['format']} {r['n']}x{r['k']}: {r['us']} us {r['GB/s']} GB/s "
              f"(cache-resident {r['cache_resident_us']} us {r['cache_resident_GB/s']} GB/s)", file=sys.stderr,
              flush=True)
    c3 = CONFIGS["9b-hybrid-q2"]
    out["cfg3_9b_hybrid"] = _generate_leg(ctx, "9B hybrid Q2_0", c3.replace(max_seq=max(c3.max_seq, 1024)), 2027,
                                          512, 129, 1.0)
    out["cfg3_9b_hybrid"]["workload"] = "9B-shaped qwen35 hybrid Q2_0, 512-token prompt, 128 greedy decode steps"
    c4 = CONFIGS["27b-hybrid-pq2"].replace(max_seq=8192)
    out["cfg4_27b_hybrid"] = _generate_leg(ctx, "27B hybrid PQ2_0", c4, 2028, 2048, 65, 1.0)
    out["cfg4_27b_hybrid"]["workload"] = ("27B-shaped qwen35 hybrid PQ2_0, 2048-token batched prefill, 64 greedy "
                                         "decode steps, 8192 context")
    return out


def hybrid_leg(ctx, n_prompt: int, K: int, W: int) -> dict:
    """The 9B-shaped qwen35 hybrid (24 Gated-DeltaNet + 8 gated-attention
    layers, Q2_0): batched prefill of an n_prompt-token prompt (the GDN layers'
    recurrence in token order on the device), then greedy decode.  The
    reference feeds hybrid prompts token by token (qwen35.rs:1693-1700)."""
    from hearth_amd import Model, CONFIGS
    cfg = CONFIGS["9b-hybrid-q2"]
    cfg = cfg.replace(max_seq=max(cfg.max_seq, n_prompt + K + W + 16))
    m = Model(ctx, cfg)
    m.synthesize(2027)
    prompt = [(i * 7919 + 13) % cfg.vocab for i in range(n_prompt)]
    m.generate(prompt[:64], 2, repeat_pen=1.0)          # warm-up (scratch, code)
    m.reset()
    toks, _ = m.generate(prompt, W + K + 1, repeat_pen=1.0)
    pf_ms = m.last_prefill_ms()
    dec_ms = m.last_decode_ms() / (W + K)
    m.close()
    print(f"[bench] 9B hybrid: prefill {n_prompt} tokens {pf_ms:.1f} ms ({n_prompt / (pf_ms * 1e-3):.0f} tok/s), "
          f"decode {dec_ms:.4f} ms/step ({1000.0 / dec_ms:.1f} tok/s)", file=sys.stderr, flush=True)
    # the same prompt through the chunked GDN recurrence (HH_GDN_CHUNKED=1):
    # fp32-rounding parity with the sequential rule, which stays the default
    os.environ["HH_GDN_CHUNKED"] = "1"
    try:
        mc = Model(ctx, cfg)
    finally:
        os.environ.pop("HH_GDN_CHUNKED", None)
    mc.synthesize(2027)
    mc.generate(prompt[:64], 2, repeat_pen=1.0)
    mc.reset()
    mc.generate(prompt, 2, repeat_pen=1.0)
    pfc_ms = mc.last_prefill_ms()
    mc.close()
    print(f"[bench] 9B hybrid, chunked GDN prefill: {n_prompt} tokens {pfc_ms:.1f} ms", file=sys.stderr, flush=True)
    # both opt-in prefill forms: chunked GDN and the fp32-MFMA attention
    os.environ["HH_GDN_CHUNKED"] = "1"
    os.environ["HH_PREFILL_ATTN"] = "mfma"
    try:
        mf = Model(ctx, cfg)
    finally:
        os.environ.pop("HH_GDN_CHUNKED", None)
        os.environ.pop("HH_PREFILL_ATTN", None)
    mf.synthesize(2027)
    mf.generate(prompt[:64], 2, repeat_pen=1.0)
    mf.reset()
    mf.generate(prompt, 2, repeat_pen=1.0)
    pff_ms = mf.last_prefill_ms()
    mf.close()
    print(f"[bench] 9B hybrid, chunked GDN + MFMA attention prefill: {n_prompt} tokens {pff_ms:.1f} ms", file=sys.stderr,
          flush=True)
    return {"model": "9B-shaped qwen35 hybrid Q2_0 (32 layers, full attention every 4th)",
            "prefill_tokens": n_prompt, "prefill_ms": round(pf_ms, 2),
            "prefill_tok_per_s": round(n_prompt / (pf_ms * 1e-3), 1),
            "decode_tok_per_s": round(1000.0 / dec_ms, 2), "decode_ms_per_step": round(dec_ms, 4),
            "prefill_chunked_gdn_ms": round(pfc_ms, 2),
            "prefill_chunked_gdn_tok_per_s": round(n_prompt / (pfc_ms * 1e-3), 1),
            "prefill_chunked_gdn_mfma_attention_ms": round(pff_ms, 2),
            "prefill_chunked_gdn_mfma_attention_tok_per_s": round(n_prompt / (pff_ms * 1e-3), 1),
            "first_tokens": [int(t) for t in toks[:8]],
            "note": "prompt through the batched prefill (bit-identical to token-by-token decode), then decode "
                    "from the prefilled state; prefill time is the prompt phase of generate"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--layers", type=int, default=0, help="override layer count (debug only)")
    ap.add_argument("--no-kv-q8", action="store_true", help="skip the Q8_0 KV-cache decode leg")
    ap.add_argument("--prefill-tokens", type=int, default=2048,
                    help="batched-prefill leg after the decode measurement (0 = skip)")
    ap.add_argument("--no-hybrid", action="store_true", help="skip the 9B hybrid prefill + decode leg")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the BASELINE configs[0,1,3,4] legs (1.7B Q1_0, GEMV microbench, 9B and 27B hybrids)")
    ap.add_argument("--hybrid-only", action="store_true",
                    help="run only the 9B hybrid leg and print its JSON (profiling)")
    ap.add_argument("--leg", choices=("1.7b", "9b", "27b", "27b-decode"), default=None,
                    help="run only one configs leg (1.7B Q1_0 = configs[0], 9B hybrid = configs[3], "
                         "27B hybrid = configs[4]; 27b-decode: the 27B at 8192 context with a 64-token "
                         "prompt and 16 decode steps, for counter runs) and print its JSON (profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs one GPU per process: bench.py measures --gpus 1 only; "
                                   "multi-GPU sharding (LM head by vocab rows, layers by pipeline stage) is not built"}))
        sys.exit(2)

    if not args.no_configs:
        # the GEMV microbench leg allocates through torch, whose bundled HIP
        # runtime must initialize before the library's (system ROCm) one
        import torch
        torch.cuda.init()
    from hearth_amd import Ctx, Model, CONFIGS
    if args.leg:
        print(json.dumps({args.leg: single_leg(Ctx(0), args.leg)}), flush=True)
        return
    if args.hybrid_only:
        print(json.dumps({"hybrid": hybrid_leg(Ctx(0), 2048, args.steps, args.warmup)}), flush=True)
        return
    cfg = CONFIGS["8b-q2"]
    if args.layers:
        cfg = cfg.replace(n_layers=args.layers)
    seed, kv_seed = 2026, 77
    K, W = args.steps, args.warmup
    cfg = cfg.replace(max_seq=max(cfg.max_seq, 2048 + max(K, W) + 8))
    ctx = Ctx(0)
    m = Model(ctx, cfg)
    m.synthesize(seed)
    m.prefill_kv_synthetic(kv_seed, 2048)
    from_seed = np.random.default_rng(seed)
    tok0 = int(from_seed.integers(0, cfg.vocab))
    print(f"[bench] model ready: 8B Q2_0, {cfg.n_layers} layers; warmup {W}, steps {K}", file=sys.stderr, flush=True)
    if W:
        m.generate([tok0], W + 1, start_pos=2048, repeat_pen=1.1)
    ctx.sync()
    t0 = time.perf_counter()
    toks, _ = m.generate([tok0], K + 1, start_pos=2048, repeat_pen=1.1)
    wall = time.perf_counter() - t0
    dev_ms = m.last_decode_ms()
    ms_per_step = dev_ms / K
    tps = 1000.0 / ms_per_step
    print(f"[bench] {K} steps: device {dev_ms:.2f} ms ({ms_per_step:.4f} ms/step), wall {wall*1e3:.1f} ms",
          file=sys.stderr, flush=True)
    mean_seq = 2048 + 1 + (K - 1) / 2.0 + 1
    b = step_bytes(cfg, int(round(mean_seq)))
    stage = m.time_stages(layer=0, iters=50)
    print(f"[bench] stage ms (layer 0): {json.dumps(stage)}", file=sys.stderr, flush=True)
    gu_ms = stage["gate_up"]
    gu_gbs = b["gate_up"] / (gu_ms * 1e-3) / 1e9
    # the kernel with the largest share of a step (rocprof ranks the
    # packed-input GEMV first: it runs twice per layer, attn_output and ffn_down)
    od_ms = stage["out_proj"] + stage["down"]
    od_bytes = b["out_proj"] + b["down"]
    od_gbs = od_bytes / (od_ms * 1e-3) / 1e9
    od_traffic = measured_traffic("void k_gemv<2, 0, 1, 1>(GemvArgs)")
    gu_traffic = measured_traffic("void k_gemv<2, 1, 2, 2>(GemvArgs)")
    step_gbs = b["total"] * tps / 1e9
    out = {
        "metric": METRIC,
        "value": round(tps, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded device-generated Q2_0/Q8_0 weights, seeded fp16-valued KV prefill)",
        "config": {"workload": "8B-shaped Q2_0 dense decoder, batch 1, KV prefilled to 2048, greedy decode",
                   "d_model": cfg.d_model, "layers": cfg.n_layers, "heads": f"{cfg.n_heads}q/{cfg.n_kv_heads}kv x {cfg.head_dim}",
                   "d_ffn": cfg.d_ffn, "vocab": cfg.vocab, "kv_dtype": "f32", "repeat_pen": 1.1,
                   "bytes_per_step": b["total"], "parallelism": "single GPU"},
        "step_hbm": {"achieved": round(step_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(step_gbs / PEAK_HBM_GBS, 4)},
        "roofline": {"bound": "hbm",
                     "kernel": "k_gemv<Q2,PACKED,ADD> (attn_output + ffn_down, layer 0; largest share of a step)",
                     "achieved": round(od_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(od_gbs / PEAK_HBM_GBS, 4),
                     "traffic": None if od_traffic is None else od_traffic,
                     "traffic_note": "mean HBM bytes per dispatch of the two launches (rocprofv3 FETCH/WRITE, "
                                     "profiles/decode_8b_q2_hbm_traffic.txt, measured on hh_gemv.hip sha256 "
                                     + gemv_source_hash() + ")" if od_traffic is not None else
                                     "null: profiles/decode_8b_q2_hbm_traffic.txt was measured on another "
                                     "version of hh_gemv.hip",
                     "avg_launch_ms": round(od_ms / 2, 5), "bytes_per_launch": od_bytes // 2},
        "roofline_gate_up": {"bound": "hbm", "kernel": "k_gemv<Q2,RMSNORM,SILU> (fused gate+up, layer 0)",
                             "achieved": round(gu_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                             "frac": round(gu_gbs / PEAK_HBM_GBS, 4), "traffic": gu_traffic,
                             "avg_launch_ms": round(gu_ms, 5), "bytes_per_launch": b["gate_up"]},
        "roofline_attention": {"bound": "hbm", "kernel": "k_attn_split + k_attn_merge (layer 0)",
                               "achieved": round(b["attention"] / (stage["mix"] * 1e-3) / 1e9, 1),
                               "peak": PEAK_HBM_GBS, "unit": "GB/s",
                               "frac": round(b["attention"] / (stage["mix"] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                               "avg_stage_ms": round(stage["mix"], 5)},
        "stage_ms": {k: round(v, 5) for k, v in stage.items()},
        "first_tokens": [int(t) for t in toks[:8]],
    }
    if not args.no_kv_q8:
        out["kv_q8"] = kv_q8_leg(ctx, cfg, seed, kv_seed, tok0, K, W)
    if args.prefill_tokens > 0:
        out["prefill"] = prefill_leg(m, cfg, args.prefill_tokens)
        out["prefill_mfma_attention"] = prefill_mfma_attention_leg(ctx, cfg, seed, args.prefill_tokens)
    if not args.no_hybrid:
        out["hybrid"] = hybrid_leg(ctx, 2048, K, W)
    if not args.no_configs:
        out["configs"] = config_legs(ctx)
    if not args.no_cpu:
        try:
            out["cpu_baseline"] = cpu_baseline(m, cfg, seed, kv_seed, tok0, args.cpu_budget)
        except Exception as e:  # the GPU number stands on its own
            out["cpu_baseline"] = {"error": repr(e)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
