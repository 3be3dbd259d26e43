"""Build liblocks_hip.so (gfx950) in-tree with hipcc.

    python locks-kv_amd/build_lib.py        # -> locks-kv_amd/locks/_lib/liblocks_hip.so

The library is plain HIP C++ behind an extern "C" ABI (include/locks_hip.h);
it links only against the HIP runtime.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "locks", "_lib")
LIB = os.path.join(OUT_DIR, "liblocks_hip.so")
SOURCES = ["locks_capi.cpp", "locks_score.hip", "locks_select.hip", "locks_decode.hip", "locks_build.hip",
           "locks_mla.hip", "locks_tier.hip",
           "locks_calib.hip"]
ARCH = "gfx950"
EXAMPLES = [("examples/capi_decode.cpp", "capi_decode")]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = ["-O3", "-fPIC", "-std=c++17", f"-I{CSRC}", f"-I{os.path.join(ROOT, 'include')}",
          "-Wall", "-Wno-unused-function"]
DEVICE = [f"--offload-arch={ARCH}", "-x", "hip",
          # packed-fp32 instructions stay off on this pool (silent wrong results)
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# per-source extra flags: the scorer keeps its MFMA accumulators in VGPRs (no
# accvgpr moves before the VALU epilogues; measured ~2 % faster).  Not for
# sources whose inline-asm LDS stores read MFMA results: the compiler's
# MFMA-to-asm wait states are only guaranteed through the accvgpr moves.
EXTRA = {"locks_score.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: str) -> str:
    obj = os.path.join(OUT_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON, *DEVICE, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    for o in objs:
        os.remove(o)
    # the C-ABI example (a non-Python host of the library), run by the GPU tests
    for src, exe in EXAMPLES:
        out = os.path.join(OUT_DIR, exe)
        cmd = [HIPCC, "-O2", "-std=c++17", f"-I{os.path.join(ROOT, 'include')}",
               f"--offload-arch={ARCH}", os.path.join(HERE, src), f"-L{OUT_DIR}", "-llocks_hip",
               "-Wl,-rpath,$ORIGIN", "-o", out + ".tmp"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
        os.replace(out + ".tmp", out)
    if verbose:
        print(f"[locks] built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
