"""Build ``libdattri_amd.so`` in-tree with hipcc for gfx950.

    python dattri-llm_amd/build.py          # or __graft_entry__.build()

Compiles every ``csrc/*.hip`` (in parallel, objects under ``_build/``) into one shared library next to the Python
package (``dattri_llm_amd/libdattri_amd.so``).  Always recompiles.
"""

from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
OUT = os.path.join(HERE, "dattri_llm_amd", "libdattri_amd.so")
OBJ_DIR = os.path.join(HERE, "_build")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wno-unused-function",
    # Inline assembly must declare every register it touches as an operand:
    # a clobber the compiler cannot honour (a reserved register such as M0)
    # fails the build instead of warning.
    "-Werror=inline-asm",
    # Packed fp32 VALU forms are kept out of the generated code.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP kernels)")


def _run(cmd: list, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{stderr}")
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile each source to an object in parallel, then link the library.

    Every ``.hip`` file is a self-contained translation unit (its kernels and
    their ``extern "C"`` launchers), so the objects link without relocatable
    device code.
    """
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    os.makedirs(OBJ_DIR, exist_ok=True)
    compile_flags = [f for f in FLAGS if f != "-shared"]
    objects = [os.path.join(OBJ_DIR, os.path.basename(s)[:-4] + ".o") for s in sources]
    jobs = jobs or min(len(sources), os.cpu_count() or 1, 16)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        futures = [pool.submit(_run, [hipcc(), *compile_flags, "-c", s, "-o", o], verbose)
                   for s, o in zip(sources, objects)]
        for f in futures:
            f.result()
    tmp = OUT + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", tmp], verbose)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
