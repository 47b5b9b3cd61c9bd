"""Build the gfx950 HIP library ``aipu_amd/libaipu_q4k.so`` in place with hipcc.

Every translation unit is compiled for gfx950 only, with
  -ffp-contract=off   (no implicit FMA: the exact kernels must round mul and add separately)
  -Xclang -target-feature -Xclang -packed-fp32-ops   (no packed fp32 VALU ops)
and linked into one shared library exposing the C ABI of include/aipu_q4k.h.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libaipu_q4k.so")
OBJDIR = os.path.join(ROOT, "_build", "obj")
ARCH = "gfx950"

SOURCES = ["abi.hip", "elementwise.hip", "router.hip", "gemv_ref.hip", "gemv_fast.hip", "moe.hip", "tiles.hip", "gemv_mfma.hip",
           "gemv_persist.hip", "gemv_persist_m.hip", "gemv_mixed.hip", "prefill.hip", "lmhead.hip", "norm.hip", "moe_batched.hip",
           "moe_persist.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
    f"-I{os.path.join(ROOT, 'include')}",
]


def hipcc():
    p = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found")
    return p


def _compile(src):
    obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    noise = [l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip()]
    return obj, "\n".join(noise)


def build(verbose=False):
    os.makedirs(OBJDIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        results = list(ex.map(_compile, SOURCES))
    for obj, warn in results:
        if warn and verbose:
            print(warn, file=sys.stderr)
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", tmp, *[o for o, _ in results]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
