"""Build the native library laii_amd/liblfm_attn.so for gfx950.

HIP translation units are compiled with hipcc (--offload-arch=gfx950), the
C11 host unit with gcc, and everything is linked into one shared library
that exports the C-ABI of include/lfm_attn.h.  Objects go to laii_amd/_build/.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "liblfm_attn.so")

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["shim.hip", "decode_splitkv.hip", "generic.hip", "prologue.hip", "prefill_fa.hip",
               "prefill_ext.hip", "kv_shift.hip", "quant_matmul.hip", "fnv_hash.hip", "peak_probe.hip"]
C_SOURCES = ["lfm_attn_host.c", "lfm_attn_ctx.c"]

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall",
    # packed-fp32 instructions stay off on this target (wrong results seen with them)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{CSRC}", f"-I{INCLUDE}",
]
# per-file additions:
# - the prefill kernels take maxima of MFMA results, which are never NaN
#   there; without the no-NaN assumption every fmaxf operand is canonicalised
#   first (one extra VALU op per score);
# - MFMA accumulators in ordinary VGPRs: for workgroups of <= 4 waves the
#   compiler otherwise puts them in AGPRs and copies them back and forth
#   around every MFMA (the decode kernels carried ~17,700 such copies; the
#   MFMA probe ran at 58 % pipe occupancy).  Same results, fewer registers:
#   e.g. k_splitkv_bal<64,2,4> 272 -> 245 VGPRs (two waves per SIMD), B1 LFM3
#   decode 44.2 -> 39.8 us, ragged B64 decode 104 -> 102.4 us on MI355X.
VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
HIP_FILE_FLAGS = {"prefill_fa.hip": ["-fno-honor-nans"], "prefill_ext.hip": ["-fno-honor-nans"],
                  "decode_splitkv.hip": VGPR_MFMA,
                  "peak_probe.hip": VGPR_MFMA}
C_FLAGS = ["-std=c11", "-O2", "-fPIC", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
           f"-I{ROCM}/include", f"-I{CSRC}", f"-I{INCLUDE}"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd[:3])} ... ({r.returncode})")
    noise = "is not a recognized feature for this target"
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if verbose and out.strip():
        print(out)


def build(verbose: bool = False) -> str:
    """Compile every source and link liblfm_attn.so; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    jobs = []
    objs = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        jobs.append([HIPCC, *HIP_FLAGS, *HIP_FILE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src),
                     "-o", obj])
        objs.append(obj)
    for src in C_SOURCES:
        obj = os.path.join(BUILD, src.replace(".c", ".o"))
        jobs.append(["gcc", *C_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        list(ex.map(lambda c: _run(c, verbose), jobs))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp, "-lm"], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
