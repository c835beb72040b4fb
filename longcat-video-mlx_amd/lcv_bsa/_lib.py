"""ctypes binding of liblcv_bsa.so (declared in include/lcv_bsa.h).

The library is loaded lazily, after torch (whose bundled HIP runtime it links
against).  A missing or unloadable library raises immediately: there is no
fallback implementation behind this module.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import c_char_p, c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "liblcv_bsa.so"

# enum lcv_bsa_dtype
F16, BF16, F32 = 0, 1, 2
# enum lcv_bsa_status
OK = 0
ERR_INVALID_ARG = 1
ERR_SHAPE = 2
ERR_DTYPE = 3
ERR_UNSUPPORTED = 4
ERR_LAYOUT = 5
ERR_LAUNCH = 6
# LCV_BSA_NOALLOC_SCRATCH_BYTES: the device array lcv_bsa_forward_noalloc holds per GPU
NOALLOC_SCRATCH_BYTES = 1 << 20


class Strides(ctypes.Structure):
    """lcv_bsa_strides: element strides of a [B, H, S, D] tensor."""

    _fields_ = [("b", c_int64), ("h", c_int64), ("s", c_int64)]


class Geom(ctypes.Structure):
    """lcv_bsa_geom: latent grid (T, Hl, Wl) and voxel (cT, cH, cW)."""

    _fields_ = [(n, c_int64) for n in ("T", "Hl", "Wl", "cT", "cH", "cW")]


class Grid(ctypes.Structure):
    """lcv_bsa_grid: latent grid (T, Hl, Wl) of the RoPE positions."""

    _fields_ = [(n, c_int64) for n in ("T", "Hl", "Wl")]


_SIGNATURES = {
    "lcv_bsa_version": (c_char_p, []),
    "lcv_bsa_strerror": (c_char_p, [c_int]),
    "lcv_bsa_last_error": (c_char_p, []),
    "lcv_bsa_pool": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_int64, Strides, Geom,
                             c_void_p, c_void_p]),
    "lcv_bsa_scores": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64,
                               c_void_p, c_void_p]),
    "lcv_bsa_topk": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p,
                             c_void_p]),
    "lcv_bsa_select": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64,
                               c_int64, c_void_p, c_void_p]),
    "lcv_bsa_schedule": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p,
                                 c_void_p]),
    "lcv_bsa_schedule_kv": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64,
                                    c_void_p, c_void_p]),
    "lcv_bsa_attn_fwd": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_int64,
                                 c_int64, Strides, Strides, Strides, c_void_p, c_void_p, c_int64,
                                 c_float, Geom, c_void_p, Strides, c_void_p]),
    "lcv_bsa_attn_fwd_kv": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_int64,
                                    c_int64, c_int64, Strides, Strides, Strides, c_void_p, c_void_p,
                                    c_int64, c_float, Geom, Geom, c_void_p, Strides, c_void_p]),
    "lcv_bsa_block_rows": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_int64, c_int64, c_int64,
                                   c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_float,
                                   c_void_p, c_void_p, c_void_p]),
    "lcv_bsa_block_swiglu": (c_int, [c_void_p, c_int, c_int64, c_int64, c_void_p, c_void_p]),
    "lcv_bsa_head_rms_norm": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_int64, Strides,
                                      c_void_p, c_float, c_void_p, Strides, c_void_p]),
    "lcv_bsa_forward_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int64, c_int64]),
    "lcv_bsa_forward": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_int64,
                                c_int64, Strides, Strides, Strides, c_int64, c_float, Geom,
                                c_void_p, c_size_t, c_void_p, c_void_p, Strides, c_void_p]),
    "lcv_bsa_forward_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_int64,
                                        c_int64, Strides, Strides, Strides, c_int64, c_float, Geom,
                                        c_void_p, c_void_p, Strides, c_void_p]),
    "lcv_bsa_token_blocks": (c_int, [Geom, c_void_p, c_void_p]),
    "lcv_bsa_token_pair_mask": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p,
                                        c_int64, c_int64, c_void_p, c_void_p]),
    "lcv_bsa_permute_block_major": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_int64,
                                            Geom, c_int, c_void_p, c_void_p]),
    "lcv_bsa_rope_table_len": (c_int64, [c_int64, Grid]),
    "lcv_bsa_prepare_qk": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_int64, c_int64, c_int64,
                                   Strides, Strides, c_void_p, c_void_p, c_float, Grid, c_void_p,
                                   c_int64, Geom, c_void_p, c_void_p, Strides, Strides, c_void_p,
                                   c_void_p, c_void_p]),
}

EXPORTED = tuple(_SIGNATURES)

_lib = None
_lock = threading.Lock()


class BSALibraryError(RuntimeError):
    """A non-shape failure reported by the native library (launch, layout...)."""


def load() -> ctypes.CDLL:
    """Load (once) and return the native library; raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m lcv_bsa._build` "
                "(or __graft_entry__.build()). The HIP backend has no fallback."
            )
        import torch  # noqa: F401  -- brings in the HIP runtime the library links against

        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def version() -> str:
    return load().lcv_bsa_version().decode()


def check(status: int, what: str) -> None:
    """Raise for a non-zero status: ValueError for contract violations (the
    reference's dense-fallback trigger), BSALibraryError otherwise."""
    if status == OK:
        return
    lib = load()
    msg = f"{what}: {lib.lcv_bsa_strerror(status).decode()}: {lib.lcv_bsa_last_error().decode()}"
    if status in (ERR_SHAPE, ERR_UNSUPPORTED, ERR_DTYPE, ERR_INVALID_ARG):
        raise ValueError(msg)
    raise BSALibraryError(msg)


__all__ = [
    "BF16", "F16", "F32", "Geom", "Grid", "Strides", "EXPORTED", "BSALibraryError", "LIB_PATH",
    "check", "load", "version",
]
