"""ctypes binding of libmegaslide_dsa3d.so (the C ABI in include/megaslide_dsa3d.h).

The library is built in-tree by ``python -m megaslide_amd.csrc.build``.  There
is no fallback: if the library is missing or a call fails, a RuntimeError says
so.  torch is imported first so that the library's libamdhip64.so.7 dependency
binds to the HIP runtime torch has already loaded (one runtime per process,
shared streams and device pointers).
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libmegaslide_dsa3d.so")
ABI_VERSION = 5

MSD_F32 = 0
MSD_BF16 = 1

# largest scratch msd_dsa3d_bwd_noalloc gives a call (MSD_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 128 << 20

# Every symbol the header declares (checked by the CPU test suite).
EXPORTS = (
    "msd_abi_version",
    "msd_last_error",
    "msd_dsa3d_fwd",
    "msd_dsa3d_bwd_workspace_size",
    "msd_dsa3d_bwd",
    "msd_dsa3d_bwd_noalloc",
    "msd_dwconv3d_fwd",
    "msd_dwconv3d_bwd_workspace_size",
    "msd_dwconv3d_bwd",
)


class DsaDesc(ctypes.Structure):
    """msd_dsa3d_desc."""

    _fields_ = [
        ("B", ctypes.c_int32), ("T", ctypes.c_int32), ("H", ctypes.c_int32), ("W", ctypes.c_int32),
        ("num_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("kt", ctypes.c_int32), ("kh", ctypes.c_int32), ("kw", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("q_stride", ctypes.c_int64), ("k_stride", ctypes.c_int64), ("v_stride", ctypes.c_int64),
        ("offset_scale", ctypes.c_float), ("softmax_scale", ctypes.c_float),
        ("algo", ctypes.c_int32), ("dropout_offset", ctypes.c_uint32),
        ("dropout_seed", ctypes.c_uint64), ("dropout_p", ctypes.c_float),
        ("extra_g", ctypes.c_int32), ("dkv_accum", ctypes.c_int32),
    ]


ALGOS = {"auto": 0, "direct": 1, "tiled": 2}

# msd_accum: how the backward sums dK / dV across query tiles
ACCUMS = {"fp32": 0, "fp16": 1}


class ConvDesc(ctypes.Structure):
    """msd_dwconv3d_desc."""

    _fields_ = [
        ("B", ctypes.c_int32), ("T", ctypes.c_int32), ("H", ctypes.c_int32), ("W", ctypes.c_int32),
        ("C", ctypes.c_int32), ("kt", ctypes.c_int32), ("kh", ctypes.c_int32), ("kw", ctypes.c_int32),
        ("dtype", ctypes.c_int32), ("act", ctypes.c_int32),
    ]


_lock = threading.Lock()
_lib = None

_vp = ctypes.c_void_p


def load() -> ctypes.CDLL:
    """Load (once) and return the library, with argtypes set."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"megaslide_amd: HIP library not built ({LIB_PATH} missing); "
                "run `python -m megaslide_amd.csrc.build`")
        lib = ctypes.CDLL(LIB_PATH)
        lib.msd_abi_version.restype = ctypes.c_int
        lib.msd_abi_version.argtypes = []
        lib.msd_last_error.restype = ctypes.c_char_p
        lib.msd_last_error.argtypes = []
        lib.msd_dsa3d_fwd.restype = ctypes.c_int
        lib.msd_dsa3d_fwd.argtypes = [ctypes.POINTER(DsaDesc)] + [_vp] * 9
        lib.msd_dsa3d_bwd_workspace_size.restype = ctypes.c_size_t
        lib.msd_dsa3d_bwd_workspace_size.argtypes = [ctypes.POINTER(DsaDesc)]
        lib.msd_dsa3d_bwd.restype = ctypes.c_int
        lib.msd_dsa3d_bwd.argtypes = [ctypes.POINTER(DsaDesc)] + [_vp] * 17 + [ctypes.c_size_t, _vp]
        lib.msd_dsa3d_bwd_noalloc.restype = ctypes.c_int
        lib.msd_dsa3d_bwd_noalloc.argtypes = [ctypes.POINTER(DsaDesc)] + [_vp] * 17
        lib.msd_dwconv3d_fwd.restype = ctypes.c_int
        lib.msd_dwconv3d_fwd.argtypes = [ctypes.POINTER(ConvDesc)] + [_vp] * 6
        lib.msd_dwconv3d_bwd_workspace_size.restype = ctypes.c_size_t
        lib.msd_dwconv3d_bwd_workspace_size.argtypes = [ctypes.POINTER(ConvDesc)]
        lib.msd_dwconv3d_bwd.restype = ctypes.c_int
        lib.msd_dwconv3d_bwd.argtypes = [ctypes.POINTER(ConvDesc)] + [_vp] * 9 + [ctypes.c_size_t, _vp]
        v = lib.msd_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"megaslide_amd: library ABI {v}, bindings expect {ABI_VERSION}")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().msd_last_error().decode(errors="replace")
        raise RuntimeError(f"megaslide_amd {what} failed (status {rc}): {msg}")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return MSD_F32
    if dt == torch.bfloat16:
        return MSD_BF16
    raise TypeError(f"megaslide_amd: dtype {dt} not supported (float32 or bfloat16)")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
