"""Builds the gfx950 library hearth_amd/libhearth_hip.so with hipcc (in-tree).

Every HIP source is compiled for gfx950 only, with packed-FP32 instructions
disabled (-packed-fp32-ops), IEEE-exact f32 division/sqrt, and no implicit
multiply-add contraction (-ffp-contract=off): element-wise arithmetic rounds
exactly like the reference's Rust code, and kernels that want a fused
multiply-add say so with fmaf().
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
SOURCES = ["hh_gemv.hip", "hh_gemm.hip", "hh_ops.hip", "hh_gdn.hip", "hh_gdn_chunk.hip", "hh_runtime.hip", "hh_gguf.cpp"]
LIB = os.path.join(HERE, "libhearth_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-fast-math", "-fhip-fp32-correctly-rounded-divide-sqrt", "-ffp-contract=off",
    "-Wall", "-Wno-unused-result", "-Wno-unused-value",
]


def build(verbose: bool = False) -> str:
    objs, cmds = [], []
    for src in SOURCES:
        obj = os.path.join(CSRC, os.path.splitext(src)[0] + ".o")
        cmds.append([HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    # one compiler process per source, at most 8 at a time
    with ThreadPoolExecutor(max_workers=min(8, len(cmds))) as pool:
        for cmd in cmds:
            if verbose:
                print(" ".join(cmd), flush=True)
        for f in [pool.submit(subprocess.run, cmd, check=True) for cmd in cmds]:
            f.result()
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", LIB]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    for o in objs:
        os.remove(o)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB)
