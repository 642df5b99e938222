"""Build libdsa_gfx950.so from the HIP sources in this directory.

Usage: ``python -m cxldsagr_amd.csrc.build`` (or ``__graft_entry__.build()``).
Compiles each ``*.hip`` file for gfx950 with hipcc and links one shared
library next to the package (``cxldsagr_amd/libdsa_gfx950.so``). No GPU is
needed; hipcc cross-compiles.
"""

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
PACKAGE = HERE.parent
ROOT = PACKAGE.parent
LIBRARY = PACKAGE / "libdsa_gfx950.so"
BUILD_DIR = ROOT / "build" / "dsa_gfx950"

ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # Packed fp32 VALU forms are disabled for all device code.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # The first kernel arguments arrive in SGPRs at wave launch (gfx950 kernarg
    # preloading; the code object keeps a 256-byte prologue that loads them
    # for firmware without it), so a kernel's first loads do not wait on the
    # kernarg segment.
    "-mllvm",
    "-amdgpu-kernarg-preload-count=16",
    f"-I{ROOT / 'include'}",
]


# Per-source device code generation flags.
# sparse_mla: MFMA accumulators in VGPRs. The O accumulators are rescaled by
# the online softmax (a VALU multiply); in AGPRs the compiler would keep a
# VGPR copy of them and move all 128 registers on every key block.
# logits: the same, plus no NaN canonicalisation around the ReLU (fmaxf would
# otherwise cost two v_max_f32 per value in a VALU-bound epilogue).
SOURCE_FLAGS = {
    "sparse_mla.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "logits.hip": ["-fno-honor-nans", "-mllvm", "-amdgpu-mfma-vgpr-form"],
    # topk: the exact row recompute of the candidate top-k runs the logits
    # arithmetic (logits_core.h) and must compile it as logits.hip does.
    "topk.hip": ["-fno-honor-nans", "-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build")
    return path


def sources():
    return sorted(HERE.glob("*.hip"))


def _compile(source):
    obj = BUILD_DIR / (source.stem + ".o")
    cmd = [hipcc(), *FLAGS, *SOURCE_FLAGS.get(source.name, []), "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{stderr}")
    return obj, stderr


def build(verbose=True):
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        results = list(pool.map(_compile, srcs))
    for obj, stderr in results:
        if verbose and stderr.strip():
            print(f"[{obj.stem}] {stderr.strip()}", file=sys.stderr)
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(obj) for obj, _ in results]]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build()
