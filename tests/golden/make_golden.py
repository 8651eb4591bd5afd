"""Writes tests/golden/golden.npz: small input/output vectors of the decode path,
computed by the CPU oracle (oracle/hearth_oracle.c) in the reference's operation
order.  The reference ships no data fixtures for this path, so these are this
repository's own; the oracle itself is pinned by the known-answer and
closed-form tests in tests/test_oracle_*.py, and these vectors then hold both
the oracle and the HIP library to fixed bytes and values.

    python tests/golden/make_golden.py        (from the repository root)

Contents (all seeded, deterministic):
  q8_x, q8_bytes          a 320-value vector with an all-zero block, a block at
                          max 127 and ties x/scale = k + 0.5, and its Q8_0 bytes
  gemv_{q1,q2,q8}_w/_a/_y 4-row GEMVs at K = 512 on the reference tests'
                          byte generators (q2_0.rs:939-986, q1_0g128.rs:1504-1551)
  dense_* / hybrid_*      2-layer dense Qwen3-style and 4-layer qwen35-style tiny
                          models (seeded synthetic weights): logits of one
                          forward at pos 0, and 32 greedy tokens after an
                          8-token prompt (repeat penalty 1.1 dense, none hybrid)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from oracle import oracle as orc            # noqa: E402
from fixtures import ref_q1_weights, ref_q2_weights, ref_act   # noqa: E402
from hearth_amd.lib import ModelConfig, GGML_Q2_0            # noqa: E402

DENSE = ModelConfig(d_model=1024, n_layers=2, n_heads=8, n_kv_heads=4, head_dim=128, d_ffn=2048,
                    vocab=4096, max_seq=128, wtype=GGML_Q2_0)
HYBRID = ModelConfig(arch=1, d_model=1024, n_layers=4, n_heads=4, n_kv_heads=2, head_dim=256, rope_dim=64,
                     d_ffn=2048, vocab=4096, max_seq=128, wtype=GGML_Q2_0, full_attn_interval=4,
                     ssm_n_k_heads=2, ssm_n_v_heads=4, ssm_head_dim=128, ssm_conv_kernel=4, attn_out_gate=1)
SEED = 2026
PROMPT = [11, 4000, 7, 123, 99, 2048, 5, 3071]


def q8_input() -> np.ndarray:
    rng = np.random.default_rng(SEED)
    x = rng.standard_normal(320).astype(np.float32)
    x[0:32] = 0.0                                   # all-zero block -> scale 1.0
    x[32] = 127.0                                    # block scale exactly 1.0 ...
    x[33:64] = np.arange(31, dtype=np.float32) - 15.5   # ... and exact .5 ties
    x[64:96] *= 1e-3
    return x


def build() -> dict:
    out = {}
    x = q8_input()
    out["q8_x"] = x
    out["q8_bytes"] = orc.quantize_q8_0(x)
    K, N = 512, 4
    for name, t, wgen, bb in (("q1", 41, ref_q1_weights, 18), ("q2", 42, ref_q2_weights, 34)):
        rows = []
        for r in range(N):   # row r: the generator's bytes with the code bytes xor (29 r)
            w = wgen(K).reshape(-1, bb)
            w[:, 2:] ^= np.uint8((29 * r) & 0xFF)
            rows.append(w.reshape(-1))
        w = np.concatenate(rows)
        a = ref_act(K, 3)
        out[f"gemv_{name}_w"], out[f"gemv_{name}_a"] = w, a
        out[f"gemv_{name}_y"] = orc.gemv(t, w, N, K, a)
    w8 = np.concatenate([ref_act(K, 5 + r) for r in range(N)])
    a8 = ref_act(K, 3)
    out["gemv_q8_w"], out["gemv_q8_a"], out["gemv_q8_y"] = w8, a8, orc.gemv(8, w8, N, K, a8)
    for name, cfg, pen in (("dense", DENSE, 1.1), ("hybrid", HYBRID, 1.0)):
        o = orc.OracleModel(cfg, seed=SEED, threads=4, order=orc.OracleModel.REFERENCE)
        out[f"{name}_logits_pos0"] = o.forward(PROMPT[0], 0)
        o.reset()
        toks, _ = o.generate(PROMPT, 32, 0, pen)
        out[f"{name}_tokens"] = toks.astype(np.uint32)
        o.close()
    out["prompt"] = np.asarray(PROMPT, dtype=np.uint32)
    out["seed"] = np.asarray([SEED], dtype=np.uint64)
    return out


if __name__ == "__main__":
    d = build()
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **d)
    print("wrote", os.path.join(HERE, "golden.npz"), sum(v.nbytes for v in d.values()), "bytes")
