"""ctypes binding of ``libdsa.so``: the C ABI declared in ``include/dsa.h``.

The structures below mirror ``dsa_fwd_args`` / ``dsa_bwd_args`` field for
field.  ``tests/test_boundary.py`` checks their sizes and offsets against the
C header compiled with gcc.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

from deberta_amd._build import LIB_PATH

DSA_F32 = 0
DSA_BF16 = 1
DSA_C2P = 1
DSA_P2C = 2
DSA_STAGE_PREP = 1
DSA_STAGE_DQ = 2
DSA_STAGE_DKDV = 4
DSA_STAGE_FOLD = 8
DSA_STAGE_TABLE = 16  # the first half of FOLD: per-offset sums (workspace)
DSA_STAGE_SUM = 32  # the second half: their fold onto dkr / dqr

EXPECTED_VERSION = 11

_i64x3 = ctypes.c_int64 * 3
_i64x2 = ctypes.c_int64 * 2


class DsaFwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("kr", ctypes.c_void_p),
        ("qr", ctypes.c_void_p),
        ("rel_table", ctypes.c_void_p),
        ("key_keep", ctypes.c_void_p),
        ("pair_keep", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("q_strides", _i64x3),
        ("k_strides", _i64x3),
        ("v_strides", _i64x3),
        ("o_strides", _i64x3),
        ("kr_strides", _i64x2),
        ("qr_strides", _i64x2),
        ("key_keep_stride_b", ctypes.c_int64),
        ("pair_keep_strides", _i64x2),
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("Lq", ctypes.c_int32),
        ("Lk", ctypes.c_int32),
        ("D", ctypes.c_int32),
        ("att_span", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("seg", ctypes.c_void_p),
        ("seg_stride_b", ctypes.c_int64),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("qc", ctypes.c_void_p),
        ("qc_strides", _i64x3),
        ("pair_keep_stride_h", ctypes.c_int64),
        ("dropout_threshold", ctypes.c_uint32),
        ("dropout_seed", ctypes.c_uint64),
        ("dropout_bits", ctypes.c_void_p),
        ("out_lo", ctypes.c_void_p),
    ]


class DsaBwdArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", DsaFwdArgs),
        ("dout", ctypes.c_void_p),
        ("do_strides", _i64x3),
        ("dq", ctypes.c_void_p),
        ("dk", ctypes.c_void_p),
        ("dv", ctypes.c_void_p),
        ("dq_strides", _i64x3),
        ("dk_strides", _i64x3),
        ("dv_strides", _i64x3),
        ("dkr", ctypes.c_void_p),
        ("dqr", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("stages", ctypes.c_int32),
        ("dtab_dtype", ctypes.c_int32),
        ("dtab_overwrite", ctypes.c_int32),
        ("dqc", ctypes.c_void_p),
        ("dqc_strides", _i64x3),
    ]


DSA_BLOCK_LN = 0
DSA_BLOCK_GELU = 1
DSA_BLOCK_RTD = 2


class DsaLnArgs(ctypes.Structure):
    """dsa_ln_args (include/dsa_block.h)."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("res", ctypes.c_void_p),
        ("gamma", ctypes.c_void_p),
        ("beta", ctypes.c_void_p),
        ("x_stride", ctypes.c_int64),
        ("res_strides", _i64x2),
        ("rows_per_group", ctypes.c_int64),
        ("y", ctypes.c_void_p),
        ("y_stride", ctypes.c_int64),
        ("mean", ctypes.c_void_p),
        ("rstd", ctypes.c_void_p),
        ("dy", ctypes.c_void_p),
        ("dy_stride", ctypes.c_int64),
        ("dz", ctypes.c_void_p),
        ("dz_stride", ctypes.c_int64),
        ("dgamma", ctypes.c_void_p),
        ("dbeta", ctypes.c_void_p),
        ("dbias", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("N", ctypes.c_int64),
        ("C", ctypes.c_int32),
        ("x_dtype", ctypes.c_int32),
        ("res_dtype", ctypes.c_int32),
        ("y_dtype", ctypes.c_int32),
        ("dy_dtype", ctypes.c_int32),
        ("dz_dtype", ctypes.c_int32),
        ("param_dtype", ctypes.c_int32),
        ("eps", ctypes.c_float),
    ]


class DsaGeluArgs(ctypes.Structure):
    """dsa_gelu_args (include/dsa_block.h)."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("dy", ctypes.c_void_p),
        ("dz", ctypes.c_void_p),
        ("dbias", ctypes.c_void_p),
        ("x_stride", ctypes.c_int64),
        ("y_stride", ctypes.c_int64),
        ("dy_stride", ctypes.c_int64),
        ("dz_stride", ctypes.c_int64),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("N", ctypes.c_int64),
        ("C", ctypes.c_int32),
        ("x_dtype", ctypes.c_int32),
        ("y_dtype", ctypes.c_int32),
        ("dy_dtype", ctypes.c_int32),
        ("dz_dtype", ctypes.c_int32),
        ("param_dtype", ctypes.c_int32),
    ]


class DsaRtdArgs(ctypes.Structure):
    """dsa_rtd_args (include/dsa_block.h)."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("b", ctypes.c_void_p),
        ("labels", ctypes.c_void_p),
        ("active", ctypes.c_void_p),
        ("x_stride", ctypes.c_int64),
        ("logits", ctypes.c_void_p),
        ("loss", ctypes.c_void_p),
        ("denom", ctypes.c_void_p),
        ("dloss", ctypes.c_void_p),
        ("dx", ctypes.c_void_p),
        ("dx_stride", ctypes.c_int64),
        ("dw", ctypes.c_void_p),
        ("db", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("N", ctypes.c_int64),
        ("C", ctypes.c_int32),
        ("x_dtype", ctypes.c_int32),
        ("dx_dtype", ctypes.c_int32),
        ("param_dtype", ctypes.c_int32),
    ]


# Entry points of include/dsa_block.h (the fused row kernels).
BLOCK_EXPORTS = (
    "dsa_block_workspace_bytes",
    "dsa_add_ln_fwd",
    "dsa_add_ln_bwd",
    "dsa_bias_gelu_fwd",
    "dsa_bias_gelu_bwd",
    "dsa_rtd_loss_fwd",
    "dsa_rtd_loss_bwd",
)

# Every entry point include/dsa.h declares.
EXPORTS = (
    "dsa_fwd",
    "dsa_bwd",
    "dsa_fwd_static",
    "dsa_bias",
    "dsa_bwd_workspace_bytes",
    "dsa_fwd_bias_bytes",
    "dsa_fwd_workspace_bytes",
    "dsa_fwd_dropout_bytes",
    "dsa_last_error",
    "dsa_version",
)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib_path() -> Path:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load ``libdsa.so`` (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: the fused disentangled-attention kernels are not built. "
                "Run `python -m deberta_amd._build` (hipcc, gfx950) first."
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.dsa_fwd.argtypes = [ctypes.POINTER(DsaFwdArgs), ctypes.c_void_p]
        lib.dsa_fwd.restype = ctypes.c_int
        lib.dsa_bwd.argtypes = [ctypes.POINTER(DsaBwdArgs), ctypes.c_void_p]
        lib.dsa_bwd.restype = ctypes.c_int
        lib.dsa_fwd_static.argtypes = [ctypes.POINTER(DsaFwdArgs), ctypes.c_void_p]
        lib.dsa_fwd_static.restype = ctypes.c_int
        lib.dsa_bias.argtypes = [ctypes.POINTER(DsaFwdArgs), ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p]
        lib.dsa_bias.restype = ctypes.c_int
        lib.dsa_bwd_workspace_bytes.argtypes = [ctypes.POINTER(DsaBwdArgs)]
        lib.dsa_bwd_workspace_bytes.restype = ctypes.c_size_t
        lib.dsa_fwd_bias_bytes.argtypes = [ctypes.POINTER(DsaFwdArgs)]
        lib.dsa_fwd_bias_bytes.restype = ctypes.c_size_t
        lib.dsa_fwd_workspace_bytes.argtypes = [ctypes.POINTER(DsaFwdArgs)]
        lib.dsa_fwd_workspace_bytes.restype = ctypes.c_size_t
        lib.dsa_fwd_dropout_bytes.argtypes = [ctypes.POINTER(DsaFwdArgs)]
        lib.dsa_fwd_dropout_bytes.restype = ctypes.c_size_t
        lib.dsa_last_error.argtypes = []
        lib.dsa_last_error.restype = ctypes.c_char_p
        lib.dsa_version.argtypes = []
        lib.dsa_version.restype = ctypes.c_int
        lib.dsa_block_workspace_bytes.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int32]
        lib.dsa_block_workspace_bytes.restype = ctypes.c_size_t
        for name, st in (
            ("dsa_add_ln_fwd", DsaLnArgs),
            ("dsa_add_ln_bwd", DsaLnArgs),
            ("dsa_bias_gelu_fwd", DsaGeluArgs),
            ("dsa_bias_gelu_bwd", DsaGeluArgs),
            ("dsa_rtd_loss_fwd", DsaRtdArgs),
            ("dsa_rtd_loss_bwd", DsaRtdArgs),
        ):
            fn = getattr(lib, name)
            fn.argtypes = [ctypes.POINTER(st), ctypes.c_void_p]
            fn.restype = ctypes.c_int
        ver = lib.dsa_version()
        if ver != EXPECTED_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {ver}, expected {EXPECTED_VERSION}; rebuild it")
        _lib = lib
        return lib


def last_error() -> str:
    msg = load().dsa_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed: {last_error()}")
