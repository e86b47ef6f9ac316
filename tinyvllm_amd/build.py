"""Build libtvattn.so (the HIP kernels + C ABI) for gfx950, in-tree.

    python -m tinyvllm_amd.build          # or: python tinyvllm_amd/build.py

Every ``csrc/*.hip`` file is compiled to an object in parallel with
``hipcc --offload-arch=gfx950`` and linked into ``tinyvllm_amd/libtvattn.so``.
The GPU code is built with packed-FP32 instructions disabled.
"""

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libtvattn.so"
INCLUDE = PKG.parent / "include"

ARCH = "gfx950"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
CFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wno-unused-result",
    f"-I{CSRC}", f"-I{INCLUDE}",
]


# Per-file flags.  The prefill kernels take maxima of scores that come out of
# the matrix cores and are never NaN for finite inputs; without NaN semantics
# the compiler emits v_max3 trees without canonicalising every operand.
FILE_FLAGS = {"flash_prefill.hip": ["-fno-honor-nans"], "flash_prefill_rows.hip": ["-fno-honor-nans"]}


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile all kernels and link ``libtvattn.so``; returns its path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = min(len(sources), max(1, min(16, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
