"""Build the gfx950 C-ABI library ``libplacemoe_amd.so`` in-tree.

Every ``csrc/*.hip`` file is compiled with ``hipcc --offload-arch=gfx950`` to an
object file (in parallel), and the objects are linked into
``placemoe_amd/_lib/libplacemoe_amd.so``.  Runs without a GPU: hipcc
cross-compiles.  Usage: ``python -m placemoe_amd.build``.

The grouped GEMM's main loop issues its buffer->LDS loads as inline asm and
counts their completion by hand (``s_waitcnt vmcnt``), out of the compiler's
sight; compiler-generated scratch traffic (register spills) inside that loop
would share the memory counter with them.  The build therefore compiles that
file with the compiler's per-kernel resource report and fails if any of its
kernels uses scratch memory or spills vector registers
(``resource_usage.json`` beside the library keeps the report).

The grouped GEMM source is compiled twice into the library: once for bf16
and once with ``-DPMX_ELT_F16`` for the fp16 entry points (``EXTRA_OBJECTS``).

Test variants: ``_lib/variants/libplacemoe_amd_<name>.so`` is the same library
with extra defines for one source (``VARIANTS``), e.g. a two-entry LDS tile
table so that the GEMM's table-overflow path runs at small shapes.
"""

from __future__ import annotations

import json
import os
import re
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

# Sources whose kernels must run without scratch memory (see the module
# docstring), and the kernel-name pattern the check applies to.
RESOURCE_CHECKED = {"grouped_gemm.hip": re.compile(r"grouped_gemm")}
RESOURCE_FLAG = "-Rpass-analysis=kernel-resource-usage"

# name -> (source, extra flags): further objects of the library, built from a
# source a second time with other defines.
#   grouped_gemm.f16: the grouped GEMM for fp16 tensors (entry points *_f16).
EXTRA_OBJECTS = {"grouped_gemm.f16": ("grouped_gemm.hip", ["-DPMX_ELT_F16"])}

# name -> (source, extra flags): library variants for tests and comparisons.
#   tiletab2: a two-entry LDS tile table (the on-the-spot tile decode runs at small shapes);
#   w8:       the eight-wave GEMM kernel for every call (the four-wave kernel switched off).
VARIANTS = {"tiletab2": ("grouped_gemm.hip", ["-DPMX_TILE_TAB=2"]),
            "w8": ("grouped_gemm.hip", ["-DPMX_GEMM_W4=0"])}
VARIANT_DIR = LIB_DIR / "variants"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; set HIPCC or install ROCm")


def library_path() -> Path:
    return LIB_DIR / LIB_NAME


def parse_resource_usage(text: str) -> list[dict]:
    """Per-kernel records from the compiler's ``kernel-resource-usage``
    remarks: name, VGPRs, AGPRs, scratch bytes per lane, VGPR and SGPR spills."""
    keys = {"VGPRs": "vgprs", "AGPRs": "agprs", "ScratchSize [bytes/lane]": "scratch",
            "VGPRs Spill": "vgpr_spill", "SGPRs Spill": "sgpr_spill"}
    out: list[dict] = []
    for line in text.splitlines():
        m = re.search(r"remark:\s+Function Name: (\S+)", line)
        if m:
            out.append({"name": m.group(1)})
            continue
        m = re.search(r"remark:\s+([A-Za-z][A-Za-z /\[\]]*?): (\d+)", line)
        if m and out and m.group(1) in keys:
            out[-1][keys[m.group(1)]] = int(m.group(2))
    return out


def check_no_scratch(records: list[dict], pattern: re.Pattern, source: str) -> None:
    """Raise if a kernel matching ``pattern`` uses scratch or spills VGPRs
    (or if the report names no such kernel, i.e. it could not be read)."""
    mine = [r for r in records if pattern.search(r["name"])]
    if not mine:
        raise RuntimeError(f"{source}: the compiler's resource report names no kernel matching {pattern.pattern}")
    bad = [r for r in mine if r.get("scratch", 0) > 0 or r.get("vgpr_spill", 0) > 0 or "scratch" not in r]
    if bad:
        lines = "\n".join(f"  {r['name']}: scratch {r.get('scratch')} B/lane, VGPR spill {r.get('vgpr_spill')}, "
                          f"VGPRs {r.get('vgprs')}, AGPRs {r.get('agprs')}" for r in bad)
        raise RuntimeError(
            f"{source}: kernels use scratch memory or spill vector registers; the hand-scheduled GEMM "
            f"pipeline assumes neither:\n{lines}"
        )


def _compile(src: Path, obj: Path, extra: list[str] | None = None) -> list[dict]:
    check = RESOURCE_CHECKED.get(src.name)
    cmd = [hipcc(), *HIP_FLAGS, *(extra or []), *([RESOURCE_FLAG] if check else []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    if not check:
        return []
    records = parse_resource_usage(proc.stderr)
    check_no_scratch(records, check, src.name)
    return records


def _link(objs: list[Path], out: Path) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)


def variant_path(name: str) -> Path:
    return VARIANT_DIR / f"libplacemoe_amd_{name}.so"


def build(verbose: bool = False) -> Path:
    """Compile every HIP source, link the shared library and the test
    variants; returns the library's path."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    VARIANT_DIR.mkdir(parents=True, exist_ok=True)
    jobs = [(s, obj_dir / (s.stem + ".o"), None) for s in sources]
    for name, (src, extra) in sorted(EXTRA_OBJECTS.items()):
        jobs.append((CSRC / src, obj_dir / f"{name}.o", extra))
    for name, (src, extra) in sorted(VARIANTS.items()):
        jobs.append((CSRC / src, obj_dir / f"{Path(src).stem}.{name}.o", extra))
    workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        reports = list(pool.map(lambda job: _compile(*job), jobs))
    objs = [o for _, o, _ in jobs[:len(sources) + len(EXTRA_OBJECTS)]]
    out = library_path()
    _link(objs, out)
    for name, (src, _) in sorted(VARIANTS.items()):
        vobjs = [obj_dir / f"{Path(src).stem}.{name}.o" if o.stem == Path(src).stem else o for o in objs]
        _link(vobjs, variant_path(name))
    usage = {job[1].name: rep for job, rep in zip(jobs, reports) if rep}
    (LIB_DIR / "resource_usage.json").write_text(json.dumps(usage, indent=1))
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
