"""Build libqbk.so (the HIP library) in-tree for gfx950.

    python quantibbler_amd/build.py          # compile every csrc/*.hip, link

Sources compile in parallel to quantibbler_amd/_build/*.o and link to
quantibbler_amd/libqbk.so, which the ctypes binding loads.  Flags:
  -O3 --offload-arch=gfx950     CDNA4 only
  -ffp-contract=off             no implicit FMA: epilogues round exactly as
                                the reference's separate multiply and add
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                no packed FP32 VALU ops (the host pass warns
                                that it does not know the feature; harmless)
Per source (EXTRA):
  decode.hip: -mllvm -amdgpu-mfma-vgpr-form=1
                                MFMA accumulators in VGPRs: the GEMV's
                                accumulators cross branches (partial load
                                steps), and in AGPRs every crossing copied
                                all sixteen of them
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libqbk.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]
EXTRA = {
    "decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [HIPCC, *CFLAGS, *EXTRA.get(os.path.basename(src), []), "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(ln for ln in (res.stderr or "").splitlines() if noise not in ln)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()
