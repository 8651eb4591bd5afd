"""GEMV microbenchmark: Q1_0 and Q2_0 GEMVs at the
1.7B shapes N x K = 6144x2048, 2048x6144, 151936x2048 on Q8_0 activations from
N(0,1), 1000 repetitions.  Each repetition reads a different weight copy from a
ring larger than 512 MB (twice the 256 MB last-level cache), so the traffic is
HBM; bytes per launch = N*(K/128)*block_bytes + (K/32)*34 + 4N.

    python -m hearth_amd.microbench [--reps 1000] [--json]
    python -m hearth_amd.microbench --copy-mb 512    (plain device copy of known
        size: the calibration run for rocprofv3 FETCH_SIZE / WRITE_SIZE counters)
"""
import argparse
import json
import sys

import numpy as np

SHAPES = [(6144, 2048), (2048, 6144), (151936, 2048)]
PEAK_GBS = 8000.0


def run(reps: int = 1000, ring_bytes: int = 600 << 20, seed: int = 1):
    import torch
    from hearth_amd import Ctx, GGML_Q1_0, GGML_Q2_0, row_bytes
    ctx = Ctx(0)
    out = []
    rng = np.random.default_rng(seed)
    for t, tname in ((GGML_Q1_0, "Q1_0"), (GGML_Q2_0, "Q2_0")):
        for n, k in SHAPES:
            wb = n * row_bytes(t, k)
            copies = max(2, -(-ring_bytes // wb))
            ring = torch.randint(0, 256, (copies, wb), dtype=torch.uint8, device="cuda")
            # finite fp16 block scales in every block
            bb = 18 if t == GGML_Q1_0 else 34
            sc = torch.tensor(np.frombuffer(np.float16(0.01).tobytes(), np.uint8), device="cuda")
            view = ring.view(copies, n * (k // 128), bb)
            view[:, :, 0] = sc[0]
            view[:, :, 1] = sc[1]
            x = torch.tensor(rng.standard_normal(k).astype(np.float32), device="cuda")
            xq = torch.zeros(k // 32 * 34, dtype=torch.uint8, device="cuda")
            y = torch.zeros(n, dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            ctx.quantize_q8_0(x, k, xq)
            for i in range(min(copies, 8)):
                ctx.gemv_q8(t, ring[i], n, k, xq, y)
            ctx.event(0)
            for i in range(reps):
                ctx.gemv_q8(t, ring[i % copies], n, k, xq, y)
            ctx.event(1)
            ms = ctx.elapsed_ms(0, 1) / reps
            nbytes = wb + (k // 32) * 34 + 4 * n
            gbs = nbytes / (ms * 1e-3) / 1e9
            out.append({"format": tname, "n": n, "k": k, "bytes": nbytes, "us": round(ms * 1e3, 3),
                        "GB/s": round(gbs, 1), "frac_peak": round(gbs / PEAK_GBS, 4), "ring_copies": copies})
            del ring
            torch.cuda.empty_cache()
    ctx.close()
    return out


def copy_calibration(mb: int, reps: int = 4) -> None:
    """reps device-to-device copies of mb MiB (torch copy kernel); each reads
    and writes exactly mb MiB."""
    import torch
    n = mb << 20
    src = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copied {mb} MiB x {reps}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=1000)
    ap.add_argument("--json", action="store_true")
    ap.add_argument("--copy-mb", type=int, default=0)
    a = ap.parse_args()
    if a.copy_mb:
        copy_calibration(a.copy_mb)
        return
    res = run(a.reps)
    if a.json:
        print(json.dumps(res))
    else:
        for r in res:
            print(f"{r['format']} {r['n']:>6}x{r['k']:<6} {r['us']:9.2f} us  {r['GB/s']:8.1f} GB/s  "
                  f"({100 * r['frac_peak']:.1f}% of {PEAK_GBS:.0f})")


if __name__ == "__main__":
    main()
