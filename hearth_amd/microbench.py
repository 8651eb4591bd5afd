"""GEMV microbenchmark: Q1_0 and Q2_0 GEMVs (and
PTQ1_0, the 28-byte ternary format) at the 1.7B shapes N x K = 6144x2048,
2048x6144, 151936x2048, plus the 8B FFN shapes, on Q8_0 activations from
N(0,1), 1000 repetitions.  Each repetition reads a different weight copy from a
ring larger than 512 MB (twice the 256 MB last-level cache), so the traffic is
HBM; bytes per launch = N*(K/128)*block_bytes + (K/32)*34 + 4N.  The same
shapes re-reading one weight copy every repetition (cache-resident, labelled
as such) are reported beside the HBM figures.

    python -m hearth_amd.microbench [--reps 1000] [--json]
    python -m hearth_amd.microbench --copy-mb 512    (plain device copy of known
        size: the calibration run for rocprofv3 FETCH_SIZE / WRITE_SIZE counters)
    python -m hearth_amd.microbench --prefill        (batched int8-MFMA GEMM at the
        27B and 8B FFN shapes, 2048 tokens, against the dense int8 MFMA peak)
"""
import argparse
import ctypes as C
import json
import sys

import numpy as np

SHAPES = [(6144, 2048), (2048, 6144), (151936, 2048), (24576, 4096), (4096, 12288)]
PEAK_GBS = 8000.0


def run(reps: int = 1000, ring_bytes: int = 600 << 20, seed: int = 1, formats=None, shapes=None):
    import torch
    from hearth_amd import Ctx, GGML_Q1_0, GGML_Q2_0, GGML_PTQ1_0, row_bytes
    ctx = Ctx(0)
    out = []
    rng = np.random.default_rng(seed)
    for t, tname in ((GGML_Q1_0, "Q1_0"), (GGML_Q2_0, "Q2_0"), (GGML_PTQ1_0, "PTQ1_0")):
        if formats is not None and tname not in formats:
            continue
        for n, k in (shapes or SHAPES):
            wb = n * row_bytes(t, k)
            copies = max(2, -(-ring_bytes // wb))
            ring = torch.randint(0, 256, (copies, wb), dtype=torch.uint8, device="cuda")
            # finite fp16 block scales in every block
            bb = {GGML_Q1_0: 18, GGML_Q2_0: 34, GGML_PTQ1_0: 28}[t]
            so = 26 if t == GGML_PTQ1_0 else 0   # scale offset in the block
            sc = torch.tensor(np.frombuffer(np.float16(0.01).tobytes(), np.uint8), device="cuda")
            view = ring.view(copies, n * (k // 128), bb)
            view[:, :, so] = sc[0]
            view[:, :, so + 1] = sc[1]
            x = torch.tensor(rng.standard_normal(k).astype(np.float32), device="cuda")
            xq = torch.zeros(k // 32 * 34, dtype=torch.uint8, device="cuda")
            y = torch.zeros(n, dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            ctx.quantize_q8_0(x, k, xq)
            # raw device addresses: the timed loop makes no torch call per launch
            wp = [ring[i].data_ptr() for i in range(copies)]
            xp, yp = xq.data_ptr(), y.data_ptr()
            for i in range(min(copies, 8)):
                ctx.gemv_q8(t, wp[i], n, k, xp, yp)
            ctx.event(0)
            for i in range(reps):
                ctx.gemv_q8(t, wp[i % copies], n, k, xp, yp)
            ctx.event(1)
            ms = ctx.elapsed_ms(0, 1) / reps
            # the same copy every repetition: served from the last-level cache
            # (and L2 where it fits), reported apart from the HBM figure
            ctx.event(0)
            for i in range(reps):
                ctx.gemv_q8(t, wp[0], n, k, xp, yp)
            ctx.event(1)
            ms_res = ctx.elapsed_ms(0, 1) / reps
            nbytes = wb + (k // 32) * 34 + 4 * n
            gbs = nbytes / (ms * 1e-3) / 1e9
            out.append({"format": tname, "n": n, "k": k, "bytes": nbytes, "us": round(ms * 1e3, 3),
                        "GB/s": round(gbs, 1), "frac_peak": round(gbs / PEAK_GBS, 4), "ring_copies": copies,
                        "cache_resident_us": round(ms_res * 1e3, 3),
                        "cache_resident_GB/s": round(nbytes / (ms_res * 1e-3) / 1e9, 1)})
            del ring
            torch.cuda.empty_cache()
    ctx.close()
    return out


PEAK_INT8_TOPS = 5000.0
PREFILL_SHAPES = [  # (label, ggml type, rows N, cols K)
    ("27B ffn gate+up PQ2_0", 142, 2 * 17408, 5120),
    ("27B ffn down PQ2_0", 142, 5120, 17408),
    ("8B ffn gate+up Q2_0", 42, 2 * 12288, 4096),
    ("1.7B ffn gate+up Q1_0", 41, 2 * 6144, 2048),
]


def prefill(tokens: int = 2048, reps: int = 5, seed: int = 3):
    """Batched GEMM time per call and int8 TOPS (2*tokens*N*K / time)."""
    import torch
    from hearth_amd import Ctx, row_bytes
    ctx = Ctx(0)
    rng = np.random.default_rng(seed)
    out = []
    for label, t, n, k in PREFILL_SHAPES:
        wb = n * row_bytes(t, k)
        w = torch.randint(0, 256, (wb,), dtype=torch.uint8, device="cuda")
        bb = 18 if t in (41, 43) else 34
        sc = torch.tensor(np.frombuffer(np.float16(0.01).tobytes(), np.uint8), device="cuda")
        view = w.view(-1, bb)
        view[:, 0] = sc[0]
        view[:, 1] = sc[1]
        xq = torch.randint(-127, 128, (tokens * (k // 32), 34), dtype=torch.int8, device="cuda").view(torch.uint8)
        s2 = torch.tensor(np.frombuffer(np.float16(0.02).tobytes(), np.uint8), device="cuda")
        xq[:, 0] = s2[0]
        xq[:, 1] = s2[1]
        y = torch.zeros(tokens * n, dtype=torch.float32, device="cuda")
        ctx.gemm_q8(t, w, n, k, xq, tokens, y)
        ctx.sync()
        ctx.event(0)
        for _ in range(reps):
            ctx.gemm_q8(t, w, n, k, xq, tokens, y)
        ctx.event(1)
        ms = ctx.elapsed_ms(0, 1) / reps
        tops = 2.0 * tokens * n * k / (ms * 1e-3) / 1e12
        out.append({"shape": label, "tokens": tokens, "n": n, "k": k, "ms": round(ms, 4),
                    "int8_TOPS": round(tops, 1), "frac_peak": round(tops / PEAK_INT8_TOPS, 4)})
        del w, xq, y
        torch.cuda.empty_cache()
    ctx.close()
    return out


def copy_bandwidth(mb: int = 1024, reps: int = 20) -> dict:
    """Measured HBM ceiling beside the published 8 TB/s: device-to-device copies
    of mb MiB (torch's copy kernel), read + written bytes per second."""
    import torch
    n = mb << 20
    src = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del src, dst
    torch.cuda.empty_cache()
    return {"MiB": mb, "ms": round(ms, 4), "GB/s": round(2 * n / (ms * 1e-3) / 1e9, 1)}


def read_bandwidth(mb: int = 2048, reps: int = 10) -> dict:
    """The read-only HBM ceiling (hh_read_bandwidth): reps passes over mb MiB,
    each lane keeping 8 16-byte loads in flight, bytes read per second."""
    from hearth_amd.lib import Ctx, _check
    ctx = Ctx(0)
    v = C.c_double()
    _check(ctx.lib.hh_read_bandwidth(ctx.h, mb << 20, reps, C.byref(v)))
    ctx.close()
    return {"MiB": mb, "GB/s": round(v.value, 1)}


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
    ap.add_argument("--prefill", action="store_true")
    a = ap.parse_args()
    if a.prefill:
        for r in prefill():
            print(json.dumps(r) if a.json else
                  f"{r['shape']:<24} {r['tokens']} x {r['n']} x {r['k']}: {r['ms']:8.3f} ms  "
                  f"{r['int8_TOPS']:7.1f} TOPS ({100 * r['frac_peak']:.1f}% of {PEAK_INT8_TOPS:.0f})")
        return
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
