"""Build the gfx950 C-ABI library ``kvserve_amd/libkvserve_amd.so`` with hipcc.

Every ``csrc/*.hip`` file is compiled separately (in parallel) and linked into one
shared library.  The library is built in-tree so it travels with the source tree.

    python -m kvserve_amd.build
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
LIB = PKG / "libkvserve_amd.so"
OBJ = PKG / "_build"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    # packed-fp32 VALU ops stay disabled on this pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the accumulators feed VALU code directly, without
    # v_accvgpr_read copies out of AGPRs
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build kvserve_amd")
    return exe


def _compile(src: Path, defines=()) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *(f"-D{d}" for d in defines), f"-I{INCLUDE}", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
    return obj


def build(verbose: bool = False, defines=()) -> Path:
    """Compile every HIP source and link the shared library; returns its path.
    `defines`: preprocessor symbols for every source (KVMI_ORDINARY_LAUNCH: the one-pass
    compress launched as an ordinary kernel, for profilers that cannot follow a
    cooperative launch; its waits are bounded either way)."""
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(lambda src: _compile(src, defines), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True, defines=["KVMI_ORDINARY_LAUNCH"] if "--ordinary-launch" in sys.argv[1:] else [])
    sys.exit(0)
