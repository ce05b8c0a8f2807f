"""ctypes binding of ``libplacemoe_amd.so`` (the C ABI in ``include/placemoe_amd.h``).

The library is loaded from ``placemoe_amd/_lib/``; a missing library raises
``RuntimeError`` - there is no fallback implementation.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

# The in-tree build; PLACEMOE_AMD_LIBRARY names another build of the same C ABI.
_DEFAULT_LIB = Path(__file__).resolve().parent / "_lib" / "libplacemoe_amd.so"
LIB_PATH = Path(os.environ.get("PLACEMOE_AMD_LIBRARY") or _DEFAULT_LIB)

PMX_OK = 0
PMX_ERR_HIP = 1
PMX_ERR_ARG = 2
PMX_ERR_SHAPE = 3
PMX_ERR_RANGE = 4

_i32p = POINTER(c_int32)
_i64p = POINTER(c_int64)

# name -> (restype, argtypes); must match include/placemoe_amd.h
SIGNATURES = {
    "pmx_version": (c_char_p, []),
    "pmx_error_string": (c_char_p, [c_int]),
    "pmx_route_workspace_bytes": (c_size_t, [c_int64, c_int32]),
    "pmx_route": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64, c_int32, c_int32,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "pmx_route_noalloc": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64, c_int32, c_int32,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "pmx_route_status": (c_int, [c_void_p, _i32p, c_void_p]),
    "pmx_moe_scatter": (c_int, [c_void_p, c_void_p, c_int64, c_int32, c_int64, c_void_p, c_void_p]),
    "pmx_moe_scatter_src": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int64, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "pmx_moe_gather": (c_int, [c_void_p, c_void_p, c_int64, c_int32, c_int64, c_void_p, c_void_p]),
    "pmx_combine_fwd": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int64, c_void_p, c_void_p]),
    "pmx_combine_bwd": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int64, c_void_p, c_void_p, c_void_p],
    ),
    "pmx_combine_bwd_top1_rows": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p],
    ),
    "pmx_segment_sum_workspace_bytes": (c_size_t, [c_int64, c_int64]),
    "pmx_segment_sum": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "pmx_gemm_fc1_swiglu_fwd": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int32, c_int64, c_int64, c_int64,
         c_void_p, c_void_p, c_void_p],
    ),
    "pmx_group_gemm_nt": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int64, c_int64, c_int64, c_void_p, c_void_p],
    ),
    "pmx_group_gemm_nt_combine_top1": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p],
    ),
    "pmx_group_gemm_nn": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int32, c_int64, c_int64, c_int64,
         c_void_p, c_void_p],
    ),
    "pmx_group_gemm_nn_unpermute_top1": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int32, c_int64, c_int64, c_int64,
         c_void_p, c_void_p, c_void_p],
    ),
    "pmx_gemm_fc2_dgrad_swiglu_bwd": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int64, c_int64, c_int64, c_void_p, c_void_p],
    ),
    "pmx_group_gemm_tn": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64,
         c_void_p],
    ),
    "pmx_weight_rows": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "pmx_swiglu_bwd_weighted": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p,
         c_void_p],
    ),
    "pmx_replica_fold": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int64, POINTER(c_float), c_int32,
         c_void_p, c_void_p],
    ),
    "pmx_replica_exchange_pack": (
        c_int,
        [c_void_p, c_int32, c_int64, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p],
    ),
    "pmx_replica_exchange_unpack": (
        c_int,
        [c_void_p, c_int32, c_int64, c_int32, c_int32, c_void_p, c_void_p, c_int32, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "pmx_route_statistics": (
        c_int,
        [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64, c_int32, c_void_p, c_void_p, c_void_p,
         c_void_p],
    ),
    "pmx_ep_payload_workspace_bytes": (c_size_t, [c_int64, c_int32]),
    "pmx_ep_dispatch_payload": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int64, c_int32, c_int32, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "pmx_ep_combine_workspace_bytes": (c_size_t, [c_int64]),
    "pmx_ep_combine_aggregate": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int32, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p],
    ),
}

# fp16 twins of the float-path entry points: the same arguments as their
# bf16 namesakes (include/placemoe_amd.h, "fp16 tensors").
F16_TWINS = (
    "pmx_moe_gather", "pmx_combine_fwd", "pmx_combine_bwd", "pmx_combine_bwd_top1_rows", "pmx_segment_sum",
    "pmx_gemm_fc1_swiglu_fwd", "pmx_group_gemm_nt", "pmx_group_gemm_nt_combine_top1", "pmx_group_gemm_nn",
    "pmx_group_gemm_nn_unpermute_top1", "pmx_gemm_fc2_dgrad_swiglu_bwd", "pmx_group_gemm_tn", "pmx_weight_rows",
    "pmx_swiglu_bwd_weighted", "pmx_replica_fold", "pmx_ep_combine_aggregate",
)
SIGNATURES.update({name + "_f16": SIGNATURES[name] for name in F16_TWINS})

_LIB = None


class PmxError(RuntimeError):
    """A C-ABI call returned an error code."""

    def __init__(self, name: str, code: int):
        self.code = code
        super().__init__(f"{name} failed: {error_string(code)} (code {code})")


def load(path: os.PathLike | None = None) -> ctypes.CDLL:
    """Load the library once and bind every signature; raises if it is missing."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    lib_path = Path(path) if path is not None else LIB_PATH
    if not lib_path.exists():
        raise RuntimeError(
            f"placemoe_amd HIP library not found at {lib_path}; build it with "
            "`python -m placemoe_amd.build` (there is no CPU fallback)."
        )
    lib = ctypes.CDLL(str(lib_path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if path is None:
        _LIB = lib
    return lib


@contextlib.contextmanager
def using(path: os.PathLike):
    """Route every call through another build of the same C ABI (a library
    variant under test) until the block ends."""
    global _LIB
    prev = _LIB
    _LIB = load(path)
    try:
        yield _LIB
    finally:
        _LIB = prev


def error_string(code: int) -> str:
    try:
        return load().pmx_error_string(int(code)).decode()
    except RuntimeError:
        return f"error {code}"


_TIMER = None  # optional callable(name) -> context manager, set by timing harnesses


def set_timer(timer) -> None:
    """Install (or clear with None) a per-call timing hook; ``timer(name)`` must
    return a context manager wrapped around every entry-point call."""
    global _TIMER
    _TIMER = timer


def call(name: str, *args) -> None:
    """Call a PMX_* returning entry point and raise on a non-zero code."""
    fn = getattr(load(), name)
    if _TIMER is None:
        rc = fn(*args)
    else:
        with _TIMER(name):
            rc = fn(*args)
    if rc != PMX_OK:
        if rc in (PMX_ERR_ARG, PMX_ERR_SHAPE):
            raise ValueError(f"{name}: {error_string(rc)} (code {rc})")
        raise PmxError(name, rc)
