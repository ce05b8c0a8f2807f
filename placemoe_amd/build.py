"""Build the gfx950 C-ABI library ``libplacemoe_amd.so`` in-tree.

Every ``csrc/*.hip`` file is compiled with ``hipcc --offload-arch=gfx950`` to an
object file (in parallel), and the objects are linked into
``placemoe_amd/_lib/libplacemoe_amd.so``.  Runs without a GPU: hipcc
cross-compiles.  Usage: ``python -m placemoe_amd.build``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "_lib"
LIB_NAME = "libplacemoe_amd.so"
OFFLOAD_ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed-fp32 VALU forms stay off: ordinary float code must not turn into
    # v_pk_{add,mul,fma}_f32.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{REPO_DIR / 'include'}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; set HIPCC or install ROCm")


def library_path() -> Path:
    return LIB_DIR / LIB_NAME


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    objs = [obj_dir / (s.stem + ".o") for s in sources]
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(lambda so: _compile(*so), zip(sources, objs)))
    out = library_path()
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
