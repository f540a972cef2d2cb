"""ctypes binding of libpnfx.so, the C ABI declared in include/pnfx.h.

The library is loaded lazily on first use and never silently replaced: if it is
missing, or a call returns an error code, a ``PnfxError`` is raised.  There is
no fallback path behind this module.
"""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpnfx.so")

ABI_VERSION = 3
PNFX_F32 = 0
PNFX_BF16 = 1
PNFX_BWD_PREPARE, PNFX_BWD_DKDV, PNFX_BWD_DQ, PNFX_BWD_ALL = 1, 2, 4, 7
PNFX_NOALLOC_SCRATCH_BYTES = 128 << 20

_lib = None


class PnfxError(RuntimeError):
    """A libpnfx.so entry point returned a non-zero status."""


def _declare(lib: ctypes.CDLL) -> None:
    i64, i32, f32, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_void_p
    sig = {
        "pnfx_abi_version": ([], i32),
        "pnfx_last_error": ([], ctypes.c_char_p),
        "pnfx_fir_fwd": ([vp, i64, i64, i64, vp, i64, i64, i64, i64, vp, i64, i32, i32, vp], i32),
        "pnfx_fir_bwd": ([vp, i64, i64, i64, vp, i64, i64, i64, i64, vp, i64, i32, i32, vp], i32),
        "pnfx_pn_rows_fwd": (
            [vp, i64, vp, i64, vp, vp, vp, i64, i64, vp, f32, f32, f32, i32, i32, i32, vp], i32),
        "pnfx_pn_rows_bwd": (
            [vp, i64, vp, i64, vp, vp, vp, vp, i64, vp, i64, i64, vp, f32, f32, f32, i32, i32,
             i32, vp], i32),
        "pnfx_flash_fwd": (
            [vp, i64, i64, i64] * 4
            + [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, vp, f32, f32, i32, i32, i32, vp],
            i32),
        "pnfx_flash_fwd_fir": (
            [vp, i64, i64, i64] * 4
            + [vp, vp, vp, vp, i64, i64, i64, i64, vp, f32, f32, i32, i32, vp, i64, i32, i32, vp],
            i32),
        "pnfx_flash_fwd_workspace_size": ([i64, i64, i64, i64], i64),
        "pnfx_flash_bwd_workspace_size": ([i64, i64, i64, i64], i64),
        "pnfx_flash_bwd": (
            [vp, i64, i64, i64] * 4
            + [vp]
            + [vp, i64, i64, i64]
            + [vp, vp, vp]
            + [vp, i64, i64, i64] * 3
            + [vp, vp, i64, i64, i64, i64, i64, vp, f32, f32, i32, i32, i32, vp], i32),
    }
    sig["pnfx_flash_bwd_stages"] = ([i32] + sig["pnfx_flash_bwd"][0], i32)
    bwd = sig["pnfx_flash_bwd"][0]  # pnfx_flash_bwd without (workspace, workspace_bytes)
    sig["pnfx_flash_bwd_noalloc"] = (bwd[:37] + bwd[39:], i32)
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res


def lib() -> ctypes.CDLL:
    """Return the loaded library, loading it on first use."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise PnfxError(
                f"{LIB_PATH} is not built; run `python -m paper_01_anti_decoy_pnfirtau_amd.build`"
            )
        handle = ctypes.CDLL(LIB_PATH)
        _declare(handle)
        if handle.pnfx_abi_version() != ABI_VERSION:
            raise PnfxError("libpnfx.so ABI version mismatch")
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().pnfx_last_error().decode(errors="replace")
        raise PnfxError(f"{what} failed ({rc}): {msg}")


def exported_symbols() -> list[str]:
    """Names of every entry point include/pnfx.h declares."""
    return [
        "pnfx_abi_version", "pnfx_last_error", "pnfx_fir_fwd", "pnfx_fir_bwd",
        "pnfx_pn_rows_fwd", "pnfx_pn_rows_bwd", "pnfx_flash_fwd", "pnfx_flash_fwd_fir",
        "pnfx_flash_fwd_workspace_size",
        "pnfx_flash_bwd_workspace_size", "pnfx_flash_bwd", "pnfx_flash_bwd_stages",
        "pnfx_flash_bwd_noalloc",
    ]
