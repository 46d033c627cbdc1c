"""Build the gfx950 HIP library `kvengine_amd/_kve.so` in-tree with hipcc.

The library links against the HIP runtime that PyTorch ships (same soname,
RPATH to torch/lib), so it shares torch's device, streams and allocations.
Run as `python -m kvengine_amd.build` or call `build()`.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "_kve.so")
BUILD_DIR = os.path.join(HERE, "_build")
ARCH = "gfx950"

SOURCES = ["kve_runtime.hip", "kve_attn.hip", "kve_kvcache.hip", "kve_lmhead.hip",
           "kve_layer.hip", "kve_linear.hip"]

# Per-file flags: the fused layer and projection kernels must round every
# product and sum like the torch ops they replace, so no multiply-add
# contraction there (the header intrinsics they call are compiled in the same
# unit).
EXTRA_FLAGS = {"kve_layer.hip": ["-ffp-contract=off"], "kve_linear.hip": ["-ffp-contract=off"]}

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # never let the compiler emit packed fp32 math
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _torch_lib() -> str:
    import torch

    return os.path.join(os.path.dirname(torch.__file__), "lib")


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return "hipcc"


def build(verbose: bool = False, jobs: int = 4) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    hipcc = _hipcc()

    def compile_one(src: str) -> str:
        obj = os.path.join(BUILD_DIR, src.replace(".hip", ".o"))
        cmd = [hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", os.path.join(CSRC, src),
               "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tlib = _torch_lib()
    tmp = OUT + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           f"-L{tlib}", "-lamdhip64", f"-Wl,-rpath,{tlib}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
