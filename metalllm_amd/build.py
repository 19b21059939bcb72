"""Builds libmetalllm_attn.so (the gfx950 kernels + C ABI) in-tree with hipcc.

    python -m metalllm_amd.build          # compile
    python -m metalllm_amd.build --stats  # also print register / LDS use per kernel

hipcc cross-compiles for gfx950 without a GPU. The packed-fp32 target feature is disabled on
purpose: every fp32 op stays scalar (v_pk_* fp32 forms are not used on this platform).
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libmetalllm_attn.so")
SOURCES = ["attn_abi.hip", "attn_fwd.hip", "attn_bwd.hip", "attn_bwd_dq.hip", "attn_bwd_dqs.hip", "attn_computed.hip",
           "attn_noalloc.hip", "sublayer.hip", "sublayer_gemm.hip", "glue.hip"]
LIBS = ["-L/opt/rocm/lib", "-lrocblas", "-Wl,-rpath,/opt/rocm/lib"]  # sublayer GEMMs

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",            # keep the reference's separate multiply/add roundings
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


# Per-source extra flags: the kernels' per-tile slot loops are fully unrolled (their register
# arrays are indexed by the slot), which exceeds the default unroll size limit.
EXTRA = {
    "attn_fwd.hip": ["-mllvm", "-pragma-unroll-threshold=200000"],
    "attn_bwd.hip": ["-mllvm", "-pragma-unroll-threshold=200000"],
    "attn_bwd_dq.hip": ["-mllvm", "-pragma-unroll-threshold=200000"],
}


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines()
                    if "unknown target feature" not in l and "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build(stats: bool = False, verbose: bool = False) -> str:
    objs, logs = [], []
    odir = os.path.join(PKG, "_build")
    os.makedirs(odir, exist_ok=True)
    for src in SOURCES:
        obj = os.path.join(odir, src + ".o")
        cmd = [HIPCC, *FLAGS, "-c", *EXTRA.get(src, [])]
        cmd = [c for c in cmd if c != "-shared"]
        if stats:
            cmd += ["-Rpass-analysis=kernel-resource-usage"]
        logs.append(_run(cmd + [os.path.join(CSRC, src), "-o", obj]))
        objs.append(obj)
    logs.append(_run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, *LIBS, "-o", LIB + ".tmp"]))
    os.replace(LIB + ".tmp", LIB)
    if stats or verbose:
        print("\n".join(l for l in logs if l))
    return LIB


if __name__ == "__main__":
    build(stats="--stats" in sys.argv, verbose=True)
    print("built", LIB)
