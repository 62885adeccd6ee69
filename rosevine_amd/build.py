"""Build the gfx950 MoE library in-tree: rosevine_amd/librvmoe.so.

Each HIP source is compiled with hipcc for gfx950 only (no other targets, no fallback paths),
with -ffp-contract=off so that only the fused operations written as fmaf are fused, and with
packed-FP32 instruction selection disabled.

`--trace` builds the diagnostic variant rosevine_amd/librvmoe_trace.so instead (RVM_PHASE_TRACE:
the decode kernels store realtime stamps; rvm_phase_trace reads them back); load it with
RVM_LIB=rosevine_amd/librvmoe_trace.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "librvmoe.so")
LIB_TRACE = os.path.join(HERE, "librvmoe_trace.so")
SOURCES = ["runtime.hip", "quant.hip", "router.hip", "decode.hip", "grouped.hip", "refops.hip", "attention.hip",
           "session.hip", "gguf.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Wall",
    "-Werror",
    "-Wno-unused-command-line-argument",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the batched kernels convert every block sum right away, and the
    # accumulation-register form costs a read per value
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def _compile(src: str, build_dir: str = BUILD, extra: tuple = ()) -> str:
    obj = os.path.join(build_dir, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass reports the device-only feature flag as unknown; that line is harmless.
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    return obj


def build(verbose: bool = False, trace: bool = False) -> str:
    build_dir, lib, extra = (BUILD + "_trace", LIB_TRACE, ("-DRVM_PHASE_TRACE",)) if trace else (BUILD, LIB, ())
    os.makedirs(build_dir, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda src: _compile(src, build_dir, extra), SOURCES))
    tmp = lib + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    return lib


if __name__ == "__main__":
    build(verbose=True, trace="--trace" in sys.argv[1:])
    sys.exit(0)
