"""Host-side check of the weight-gradient K-tile window arithmetic
(``placemoe_amd/csrc/ktile.h``), compiled with the host compiler.

For a group of R rows of ``row_bytes`` each, K-tile kt must cover exactly
rows [64 kt, min(64 kt + 64, R)): its window starts at byte 64 kt row_bytes
of the group, and every byte of those rows lies inside the window.  Python's
integers do not wrap, so groups larger than 4 GiB (where 32-bit offsets
would wrap and the descriptor would end early) are checked exactly.
"""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
MAX_DESCRIPTOR = 2**31 - 1


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        pytest.skip("no host C++ compiler")
    exe = tmp_path_factory.mktemp("ktile") / "ktile_window"
    subprocess.run([cxx, "-O2", "-std=c++17", f"-I{ROOT / 'placemoe_amd' / 'csrc'}",
                    str(ROOT / "tests" / "ktile_window_main.cpp"), "-o", str(exe)], check=True)
    return exe


@pytest.mark.parametrize("rows,row_bytes", [
    (1, 16), (63, 4096), (64, 4096), (19421, 14336),  # config 3's largest copy, H = 7168
    (160_000, 14336),  # 2.3 GB: past one descriptor's 2 GiB
    (300_000, 14336),  # 4.3 GB: past 32-bit offsets
    (1_000_000, 8192),  # 8.2 GB, rows of 4096 bf16 (fc1 gradient rows at I = 2048)
])
def test_every_ktile_window_covers_its_rows(driver, rows, row_bytes):
    out = subprocess.run([str(driver), str(rows), str(row_bytes)], check=True, capture_output=True,
                         text=True).stdout.split("\n")
    group_bytes = rows * row_bytes
    lines = [line.split() for line in out if line and not line.startswith("dead")]
    nk = -(-rows // 64)
    assert len(lines) == nk + 1
    for kt_s, off_s, nbytes_s in lines:
        kt, off, nbytes = int(kt_s), int(off_s), int(nbytes_s)
        assert off == kt * 64 * row_bytes, f"K-tile {kt}: window starts at byte {off}"
        need_rows = max(0, min(64, rows - 64 * kt))
        assert need_rows * row_bytes <= nbytes, f"K-tile {kt}: window of {nbytes} B misses its rows"
        assert nbytes == min(max(group_bytes - off, 0), MAX_DESCRIPTOR), f"K-tile {kt}: window size {nbytes}"
        if kt == nk:
            assert nbytes == 0, "the window past the group's end must be empty"
    dead = [line.split() for line in out if line.startswith("dead")]
    assert dead == [["dead", "0", "0"]], "a dead pipeline slot must load nothing"
