"""ctypes binding of libdsqg_hip.so (the C ABI in include/dsqg.h).

The structures below mirror the header field for field.  Loading the library needs only the
HIP runtime (present on a CPU-only host too); launching needs a GPU.  There is no fallback:
if the library is missing, every entry point raises.
"""

from __future__ import annotations

import ctypes
import functools
import os
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("DSQG_HIP_LIB", PKG_DIR / "libdsqg_hip.so"))

MAX_OFFSETS = 64
ABI_VERSION = 3

DSQG_OK, DSQG_EINVAL, DSQG_EUNSUPPORTED, DSQG_EHIP, DSQG_EWORKSPACE = 0, 1, 2, 3, 4
DSQG_ETOOLARGE = 5
NOALLOC_SCRATCH_BYTES = 64 << 20  # DSQG_NOALLOC_SCRATCH_BYTES
DSQG_F32, DSQG_BF16, DSQG_F16 = 0, 1, 2

_i64x4 = ctypes.c_int64 * 4
_vp = ctypes.c_void_p


class Shape(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("B", ctypes.c_int32), ("H", ctypes.c_int32),
                ("N", ctypes.c_int32), ("D", ctypes.c_int32), ("J", ctypes.c_int32),
                ("offsets", ctypes.c_int32 * MAX_OFFSETS)]


class FwdArgs(ctypes.Structure):
    _fields_ = [("shape", Shape),
                ("q", _vp), ("q_stride", _i64x4),
                ("k", _vp), ("k_stride", _i64x4),
                ("v", _vp), ("v_stride", _i64x4),
                ("pos_bias", _vp), ("scale_embed", _vp), ("score_gain", _vp), ("if_gain", _vp),
                ("out", _vp), ("out_stride", _i64x4),
                ("lse", _vp), ("alpha_lr", _vp)]


class BwdArgs(ctypes.Structure):
    _fields_ = [("shape", Shape),
                ("q", _vp), ("q_stride", _i64x4),
                ("k", _vp), ("k_stride", _i64x4),
                ("v", _vp), ("v_stride", _i64x4),
                ("dout", _vp), ("dout_stride", _i64x4),
                ("lse", _vp),
                ("pos_bias", _vp), ("scale_embed", _vp), ("score_gain", _vp), ("if_gain", _vp),
                ("dq", _vp), ("dq_stride", _i64x4),
                ("dk", _vp), ("dk_stride", _i64x4),
                ("dv", _vp), ("dv_stride", _i64x4),
                ("dpos_bias", _vp), ("dscale_embed", _vp), ("dscore_gain", _vp),
                ("dif_gain", _vp),
                ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
                ("alpha_lr", _vp)]


class DecodeArgs(ctypes.Structure):
    _fields_ = [("shape", Shape), ("S", ctypes.c_int32),
                ("q", _vp), ("k_new", _vp), ("v_new", _vp), ("k_ring", _vp), ("v_ring", _vp),
                ("pos", _vp), ("pos_next", _vp),
                ("pos_bias", _vp), ("scale_embed", _vp), ("score_gain", _vp), ("if_gain", _vp),
                ("out", _vp)]


_i64x2 = ctypes.c_int64 * 2


class PoolFwdArgs(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("N", ctypes.c_int32), ("C", ctypes.c_int32),
                ("x_dtype", ctypes.c_int32), ("gate_dtype", ctypes.c_int32),
                ("out_dtype", ctypes.c_int32),
                ("x", _vp), ("x_stride", _i64x2),
                ("gate_pre", _vp), ("gate_stride", _i64x2),
                ("out", _vp), ("out_stride", _i64x2),
                ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t)]


class PoolBwdArgs(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("N", ctypes.c_int32), ("C", ctypes.c_int32),
                ("x_dtype", ctypes.c_int32), ("gate_dtype", ctypes.c_int32),
                ("dout_dtype", ctypes.c_int32),
                ("x", _vp), ("x_stride", _i64x2),
                ("gate_pre", _vp), ("gate_stride", _i64x2),
                ("dout", _vp), ("dout_stride", _i64x2),
                ("dx", _vp), ("dx_stride", _i64x2),
                ("dgate_pre", _vp), ("dgate_stride", _i64x2),
                ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t)]


# Every symbol include/dsqg.h declares, with its ctypes signature.
SIGNATURES = {
    "dsqg_abi_version": (ctypes.c_int, []),
    "dsqg_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "dsqg_supported_head_dims": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int32), ctypes.c_int]),
    "dsqg_fwd": (ctypes.c_int, [ctypes.POINTER(FwdArgs), _vp]),
    "dsqg_long_range_taps": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int32), ctypes.c_int]),
    "dsqg_alpha_lr_elems": (ctypes.c_int, [ctypes.POINTER(Shape), ctypes.POINTER(ctypes.c_size_t)]),
    "dsqg_bwd_workspace_size": (ctypes.c_int, [ctypes.POINTER(BwdArgs),
                                               ctypes.POINTER(ctypes.c_size_t)]),
    "dsqg_bwd": (ctypes.c_int, [ctypes.POINTER(BwdArgs), _vp]),
    "dsqg_bwd_dq": (ctypes.c_int, [ctypes.POINTER(BwdArgs), _vp]),
    "dsqg_bwd_dkdv": (ctypes.c_int, [ctypes.POINTER(BwdArgs), _vp]),
    "dsqg_bwd_params": (ctypes.c_int, [ctypes.POINTER(BwdArgs), _vp]),
    "dsqg_bwd_noalloc": (ctypes.c_int, [ctypes.POINTER(BwdArgs), _vp]),
    "dsqg_decode_step": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), _vp]),
    "dsqg_pool_gate_workspace_size": (ctypes.c_int, [ctypes.c_int32, ctypes.c_int32,
                                                     ctypes.c_int32, ctypes.c_int,
                                                     ctypes.POINTER(ctypes.c_size_t)]),
    "dsqg_pool_gate_fwd": (ctypes.c_int, [ctypes.POINTER(PoolFwdArgs), _vp]),
    "dsqg_pool_gate_bwd": (ctypes.c_int, [ctypes.POINTER(PoolBwdArgs), _vp]),
}

_LIB = None


class DSQGLibraryError(RuntimeError):
    """The HIP library is missing, stale, or returned a non-OK status."""


def load() -> ctypes.CDLL:
    """Load libdsqg_hip.so once; raise if it is missing or its ABI version differs."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise DSQGLibraryError(
            f"{LIB_PATH} is missing: build it with `python -m dwarf_amd.build` "
            "(there is no CPU fallback)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.dsqg_abi_version()
    if ver != ABI_VERSION:
        raise DSQGLibraryError(f"{LIB_PATH} has ABI version {ver}, expected {ABI_VERSION}")
    _LIB = lib
    return lib


def status_string(code: int) -> str:
    return load().dsqg_status_string(code).decode()


def check(code: int, what: str) -> None:
    if code != DSQG_OK:
        raise DSQGLibraryError(f"{what} failed: status {code} ({status_string(code)})")


def supported_head_dims() -> list[int]:
    buf = (ctypes.c_int32 * 16)()
    n = load().dsqg_supported_head_dims(buf, 16)
    return [buf[i] for i in range(min(n, 16))]


def make_shape(dtype_code: int, B: int, H: int, N: int, D: int, offsets) -> Shape:
    """A dsqg_shape block: a copy of a cached one (filling the 64-entry offset table from
    Python costs more than the copy)."""
    return Shape.from_buffer_copy(_shape_cached(dtype_code, B, H, N, D, tuple(int(o) for o in offsets)))


@functools.lru_cache(maxsize=256)
def _shape_cached(dtype_code: int, B: int, H: int, N: int, D: int, offsets: tuple) -> Shape:
    offs = list(offsets)
    if not 1 <= len(offs) <= MAX_OFFSETS:
        raise ValueError(f"offset table must have 1..{MAX_OFFSETS} entries, got {len(offs)}")
    s = Shape()
    s.dtype, s.B, s.H, s.N, s.D, s.J = dtype_code, B, H, N, D, len(offs)
    for i, o in enumerate(offs):
        s.offsets[i] = int(o)
    return s


def long_range_taps(offsets) -> int:
    """Taps beyond the dense window of an offset table (the NS of the forward's alpha_lr)."""
    arr = (ctypes.c_int32 * len(offsets))(*offsets)
    ns = load().dsqg_long_range_taps(arr, len(offsets))
    if ns < 0:
        raise DSQGLibraryError(f"dsqg_long_range_taps: {status_string(-ns)}")
    return ns
