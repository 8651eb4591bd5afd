"""Teacher-forced greedy-token comparison against the reference-order oracle.

The reference sequence is the one the reference-order oracle generates
greedily (its own tokens).  Every candidate (the HIP library, or the oracle in
the device's fp32 order) is fed that same sequence, one token per step, and
must pick the same greedy token at every step.  Where it picks another token,
the step is accepted only if the reference-order logits rank the two tokens
closer than the spread between the reference's own two CPU arms on the same
run: the scalar DotFn arm and the AVX2 arm (q2_0.rs:308-392 / :537-574), whose
fp32 groupings differ as the device's does.  The spread is the largest
|logit_scalar - logit_avx2| over every step of the run.

Dense models may run with a repetition penalty: then a step's token is the
sampler's (hearth-sampler lib.rs:26-40 + :156-207, via the oracle's
ho_sample_greedy_dense) over the penalized logits, with past tokens = the last
prompt token and every generated token (mod.rs:2879, :2949), and the gap is
measured on the penalized reference logits.
"""
import ctypes as C

import numpy as np


def argmax_first(x):
    """qwen35.rs:1735-1745: strict > scan, first maximal index."""
    return int(np.argmax(x))


def argmax_last(x):
    """hearth-sampler lib.rs:156-207 max_by: last maximal index."""
    return int(len(x) - 1 - np.argmax(x[::-1]))


def _penalized(oracle, logits, past, pen):
    x = np.array(logits, dtype=np.float32)
    if pen == 1.0:
        return x
    p = np.ascontiguousarray(np.asarray(past, dtype=np.uint32))
    oracle.load().ho_sample_greedy_dense(x.ctypes.data, x.size, p.ctypes.data, p.size, C.c_float(pen))
    return x


def _pick(oracle, cfg, logits, past, pen):
    if cfg.arch == 1:
        return argmax_first(logits)
    return argmax_last(_penalized(oracle, logits, past, pen))


def reference_run(oracle, cfg, seed, prompt, n_gen, threads=4, pen=1.0, prefilled=0, kv_seed=None):
    """Reference-order greedy run: returns the full token sequence, per-step
    reference logits (scalar arm, penalized when pen != 1) and the arm spread.
    Also leaves on the function the scalar arm's raw per-step logits
    (`raw_logits`) and the AVX2 arm's relative deviation from them (`avx_rel`,
    max |avx - scalar| / max |scalar|, same teacher-forced inputs).
    `prefilled` > 0 starts at that position over a synthetic KV cache."""
    ref = oracle.OracleModel(cfg, seed=seed, threads=threads, arm=0, order=oracle.OracleModel.REFERENCE)
    avx = oracle.OracleModel(cfg, seed=seed, threads=threads, arm=1, order=oracle.OracleModel.REFERENCE)
    if prefilled:
        ref.prefill_kv_synthetic(kv_seed, prefilled)
        avx.prefill_kv_synthetic(kv_seed, prefilled)
    seq = list(prompt)
    past = [prompt[-1]]
    logits, spread = [], 0.0
    avx_div = 0
    raw, avx_rel = [], []
    for i in range(len(prompt) + n_gen - 1):
        pos = prefilled + i
        need = i >= len(prompt) - 1
        lr = ref.forward(seq[i], pos) if need else ref.lib.ho_forward(ref.h, seq[i], pos, None)
        if need:
            la = avx.forward(seq[i], pos)
            spread = max(spread, float(np.abs(lr.astype(np.float64) - la).max()))
            raw.append(np.array(lr, dtype=np.float32))
            avx_rel.append(float(np.abs(la.astype(np.float64) - lr).max() / np.abs(lr).max()))
            logits.append(_penalized(oracle, lr, past, pen))
            tok = _pick(oracle, cfg, lr, past, pen)
            avx_div += int(_pick(oracle, cfg, la, past, pen) != tok)
            seq.append(tok)
            past.append(tok)
        else:
            avx.lib.ho_forward(avx.h, seq[i], pos, None)
    ref.close()
    avx.close()
    reference_run.avx_divergences = avx_div
    reference_run.raw_logits = raw
    reference_run.avx_rel = avx_rel
    return seq, logits, spread


def ambiguous_steps(ref_logits, spread):
    """Steps whose reference top-2 gap is below the arm spread: the only steps
    at which a divergence is accepted."""
    n = 0
    for lr in ref_logits:
        top2 = np.partition(np.asarray(lr, np.float64), -2)[-2:]
        n += int(top2[1] - top2[0] <= spread)
    return n


def check_candidate(cfg, seq, ref_logits, spread, n_prompt, forward, oracle=None, pen=1.0, prefilled=0):
    """forward(token, pos) -> logits of the candidate.  Returns the list of
    (step, ref_token, cand_token, gap) divergences; raises AssertionError if a
    divergence is not explained by the arm spread."""
    out = []
    step = 0
    past = [seq[n_prompt - 1]]
    for i in range(len(seq) - 1):
        lg = forward(seq[i], prefilled + i)
        if i < n_prompt - 1:
            continue
        want = seq[i + 1]
        got = _pick(oracle, cfg, lg, past, pen)
        past.append(want)
        if got != want:
            lr = ref_logits[step].astype(np.float64)
            gap = float(lr[want] - lr[got])
            out.append((step, want, got, gap))
            assert gap <= spread, f"step {step}: token {got} != {want}, reference gap {gap:.3g} > arm spread {spread:.3g}"
        step += 1
    return out
