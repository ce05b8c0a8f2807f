"""The C-ABI library loads without a GPU and exports every entry point that
include/placemoe_amd.h declares, with the binding table in sync."""

import ctypes
import re
from pathlib import Path

import pytest

from placemoe_amd import _capi, build

HEADER = Path(__file__).resolve().parents[1] / "include" / "placemoe_amd.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pmx_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("compiler,lang", [("gcc", "c"), ("g++", "c++")])
def test_header_compiles_standalone(compiler, lang, tmp_path):
    """A binding written against the header alone (cgo, ctypes generators, C
    callers) must be able to include it: plain C and C++, no HIP headers."""
    import shutil
    import subprocess

    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} not available")
    src = tmp_path / ("t.c" if lang == "c" else "t.cpp")
    src.write_text(f'#include "{HEADER}"\nint main(void) {{ return pmx_version() != 0 ? 0 : 1; }}\n')
    proc = subprocess.run([compiler, "-fsyntax-only", "-Wall", "-Werror", "-x", lang, str(src)],
                          capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr


def test_header_declares_the_path():
    names = declared_functions()
    for must in ("pmx_route", "pmx_moe_scatter", "pmx_gemm_fc1_swiglu_fwd", "pmx_group_gemm_tn",
                 "pmx_combine_fwd", "pmx_combine_bwd", "pmx_replica_fold"):
        assert must in names


def test_library_exports_every_declared_symbol():
    if not _capi.LIB_PATH.exists():
        build.build()
    lib = ctypes.CDLL(str(_capi.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"missing exports: {missing}"


def test_binding_table_matches_header():
    assert sorted(_capi.SIGNATURES) == declared_functions()


def test_host_only_calls_without_gpu():
    lib = _capi.load()
    assert b"gfx950" in lib.pmx_version()
    assert lib.pmx_error_string(_capi.PMX_ERR_SHAPE) == b"unsupported shape"
    assert lib.pmx_route_workspace_bytes(131072, 160) >= 256 + 64 * 160 * 4
    assert lib.pmx_route_workspace_bytes(-1, 4) == 0


def test_argument_errors_are_codes_not_crashes():
    lib = _capi.load()
    # invalid sizes are rejected before any device work
    assert lib.pmx_route(None, None, None, 0, 1, 1, 4, 2, 0, None, None, None, None, None, 0, None) == _capi.PMX_ERR_ARG
    assert lib.pmx_group_gemm_nt(None, None, None, 0, 8, 8, 8, None, None) == _capi.PMX_ERR_ARG
    assert lib.pmx_group_gemm_nt(None, None, None, 4, 8, 12, 8, None, None) == _capi.PMX_ERR_SHAPE
    assert lib.pmx_combine_bwd(None, None, None, None, 4, 33, 8, None, None, None) == _capi.PMX_ERR_ARG
    dummy = ctypes.c_void_p(16)
    assert lib.pmx_combine_bwd_top1_rows(None, None, None, None, 4, 8, None, None, None) == _capi.PMX_ERR_ARG
    assert lib.pmx_combine_bwd_top1_rows(dummy, dummy, dummy, dummy, -1, 8, dummy, dummy, None) == _capi.PMX_ERR_ARG
    assert lib.pmx_combine_bwd_top1_rows(dummy, dummy, dummy, dummy, 4, 12, dummy, dummy, None) == _capi.PMX_ERR_SHAPE
    assert lib.pmx_combine_bwd_top1_rows(dummy, dummy, dummy, dummy, 0, 8, dummy, dummy, None) == _capi.PMX_OK
    assert lib.pmx_weight_rows(None, None, 4, 8, None, None) == _capi.PMX_ERR_ARG
    assert lib.pmx_weight_rows(dummy, dummy, -1, 8, dummy, None) == _capi.PMX_ERR_ARG
    assert lib.pmx_weight_rows(dummy, dummy, 0, 8, dummy, None) == _capi.PMX_OK
    assert lib.pmx_weight_rows(dummy, dummy, 1 << 62, 8, dummy, None) == _capi.PMX_ERR_SHAPE
    swb = lib.pmx_swiglu_bwd_weighted
    assert swb(dummy, dummy, dummy, dummy, dummy, 4, 8, 4, dummy, None, None) == _capi.PMX_ERR_ARG  # dw without row_src
    assert swb(dummy, dummy, dummy, dummy, None, 4, 8, 4, dummy, dummy, None) == _capi.PMX_ERR_ARG
    assert swb(None, None, None, None, None, 4, 8, 0, None, None, None) == _capi.PMX_ERR_ARG
    assert swb(dummy, dummy, dummy, dummy, dummy, 4, -8, 4, dummy, dummy, None) == _capi.PMX_ERR_ARG
    assert swb(dummy, dummy, dummy, dummy, dummy, 0, 8, 0, dummy, dummy, None) == _capi.PMX_OK
    assert swb(dummy, dummy, dummy, dummy, dummy, 1 << 40, 8, 4, dummy, dummy, None) == _capi.PMX_ERR_SHAPE
    with pytest.raises(ValueError):
        _capi.call("pmx_group_gemm_nt", None, None, None, 4, 8, 12, 8, None, None)


def test_size_limits_rejected_before_any_launch():
    """Shapes beyond the 32-bit row and position indices are refused on the
    host (PMX_ERR_SHAPE) before any HIP call, so this runs without a GPU."""
    lib = _capi.load()
    big = 1 << 31
    dummy = ctypes.c_void_p(16)
    ws = ctypes.c_void_p(16)
    assert lib.pmx_moe_scatter(dummy, dummy, big, 1, 64, dummy, None) == _capi.PMX_ERR_SHAPE
    assert lib.pmx_moe_gather(dummy, dummy, big // 8, 8, 64, dummy, None) == _capi.PMX_ERR_SHAPE
    assert lib.pmx_combine_fwd(dummy, dummy, dummy, big, 1, 64, dummy, None) == _capi.PMX_ERR_SHAPE
    assert lib.pmx_combine_bwd(dummy, dummy, dummy, dummy, big // 2, 2, 64, dummy, dummy, None) == _capi.PMX_ERR_SHAPE
    assert lib.pmx_route(dummy, None, None, 0, 0, 0, big // 4, 4, 8, dummy, dummy, dummy, dummy, ws, 1 << 40,
                         None) == _capi.PMX_ERR_SHAPE
    assert lib.pmx_group_gemm_nt(dummy, dummy, dummy, 1, big, 64, 64, dummy, None) == _capi.PMX_ERR_SHAPE
    # argument errors
    assert lib.pmx_moe_scatter(dummy, dummy, -1, 1, 64, dummy, None) == _capi.PMX_ERR_ARG
    assert lib.pmx_replica_exchange_pack(dummy, 7, 64, 4, 1, dummy, dummy, dummy, dummy, dummy, None) == \
        _capi.PMX_ERR_ARG
    assert lib.pmx_replica_exchange_unpack(dummy, 0, 64, 4, 1, dummy, dummy, 1, dummy, None, None, None, dummy,
                                           None) == _capi.PMX_ERR_ARG


def test_wgrad_output_layout_rejected_before_any_launch():
    """The weight gradient's output copies must be 16-byte aligned, 8-element
    strided and must not overlap; each mistake is refused on the host."""
    lib = _capi.load()
    p = ctypes.c_void_p(256)
    tn = lib.pmx_group_gemm_tn
    M, N, G, K = 64, 64, 2, 128
    assert tn(p, p, p, G, K, M, N, ctypes.c_void_p(258), None, M * N, 0, None) == _capi.PMX_ERR_SHAPE
    assert tn(p, p, p, G, K, M, N, p, None, M * N + 4, 0, None) == _capi.PMX_ERR_SHAPE
    assert tn(p, p, p, G, K, M, N, p, None, M * N - 8, 0, None) == _capi.PMX_ERR_ARG
    assert tn(p, p, p, G, K, M, N, p, ctypes.c_void_p(264), (M // 2) * N, M // 2, None) == _capi.PMX_ERR_SHAPE
    assert tn(p, p, p, G, K, M, N, p, p, (M // 2) * N, 0, None) == _capi.PMX_ERR_ARG
    assert tn(p, p, p, G, K, M, N, p, p, (M // 2) * N, M, None) == _capi.PMX_ERR_ARG
    assert tn(p, p, p, G, K, M, N, p, p, (M // 2) * N - 8, M // 2, None) == _capi.PMX_ERR_ARG


def test_fc1_n_tiles_beyond_the_tile_table_rejected_before_any_launch():
    """A tile's n-index is packed in 19 bits of the kernel's LDS tile table:
    fc1 shapes with 2^19 or more 128-column n-tiles (I >= 2^26) are refused
    on the host with PMX_ERR_SHAPE, before the device is touched."""
    lib = _capi.load()
    p = ctypes.c_void_p(256)
    H, I = 8, 1 << 26
    rc = lib.pmx_gemm_fc1_swiglu_fwd(p, p, p, 2 * I * H, p, 1, 256, H, I, p, p, None)
    assert rc == _capi.PMX_ERR_SHAPE
