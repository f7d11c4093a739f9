"""Build recipe for the HIP extension ``libdsa_mi355x.so`` (gfx950).

Each ``csrc/*.hip`` file is compiled with hipcc for gfx950 in parallel, then linked into
one shared library next to this file.  No torch headers are involved: the library is a
plain C ABI (``include/dsa_mi355x.h``) loaded with ctypes.

    python -m torchtitan_npu_simulator_amd.build          # or: __graft_entry__.build()
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
BUILD_DIR = REPO_DIR / "_build"
LIB_PATH = PKG_DIR / "libdsa_mi355x.so"
ARCH = os.environ.get("DSA_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-munsafe-fp-atomics",
    # packed fp32 VALU ops are kept off on this target (they are generated from scalar
    # float code and have produced wrong results on these boxes)
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the DSA HIP extension)")


# per-source additions: the backward's score kernel keeps Q and dO in AGPRs as MFMA operands
# and its accumulators in VGPRs (read by the softmax every block)
EXTRA_FLAGS = {
    "sparse_mla_bwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: Path, obj: Path) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o",
           str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")


def build(verbose: bool = True) -> Path:
    """Compile every HIP source and link ``libdsa_mi355x.so``; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objs = [BUILD_DIR / (s.stem + ".o") for s in sources]
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda so: _compile(*so), zip(sources, objs)))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[dsa build] {len(sources)} sources -> {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build()
    sys.exit(0)
