"""ctypes binding of libspectra_hip.so (the C ABI declared in include/spectra_hip.h).

The library is built in-tree by ``python -m spectra_amd._build``.  There is no
fallback: if the library is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from ctypes import c_int32, c_int64, c_size_t, c_void_p, c_char_p

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libspectra_hip.so")
TORCH_OPS_PATH = os.path.join(_PKG, "_spectra_torch.so")

# spectra_status_t / dtype / format / outlier enums (include/spectra_hip.h)
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP, ERR_WORKSPACE = 0, -1, -2, -3, -4
F16, BF16, F32 = 0, 1, 2
FMT_ASYM_G32, FMT_NF4 = 0, 1
OUTLIERS_NONE, OUTLIERS_COLUMNS, OUTLIERS_CSR = 0, 1, 2


class QWeight(ctypes.Structure):
    """Mirror of ``spectra_qweight_t``."""
    _fields_ = [
        ("n", c_int64), ("k", c_int64),
        ("format", c_int32), ("group_size", c_int32), ("hadamard_block", c_int32), ("marlin_layout", c_int32),
        ("packed", c_void_p), ("packed_stride", c_int64),
        ("scales", c_void_p), ("scales_stride", c_int64),
        ("zeros", c_void_p), ("zeros_stride", c_int64),
        ("outlier_kind", c_int32), ("num_outliers", c_int32),
        ("outlier_idx", c_void_p),
        ("outlier_w", c_void_p), ("outlier_w_stride", c_int64),
        ("outlier_w_dtype", c_int32),
        ("csr_rowptr", c_void_p), ("csr_col", c_void_p), ("csr_val", c_void_p),
        ("csr_nnz", c_int64),
        ("bias", c_void_p), ("bias_dtype", c_int32),
    ]


PROLOGUE_NONE, PROLOGUE_RMSNORM, PROLOGUE_SILU_MUL = 0, 1, 2
ARGMAX_SLOTS, ARGMAX_STRIDE = 256, 32  # SPECTRA_ARGMAX_SLOTS, SPECTRA_ARGMAX_STRIDE


class GemvFusion(ctypes.Structure):
    """Mirror of ``spectra_gemv_fusion_t``."""
    _fields_ = [("prologue", c_int32), ("eps", ctypes.c_float), ("norm_weight", c_void_p),
                ("residual", c_void_p), ("residual_stride", c_int64), ("argmax_key", c_void_p)]


# name -> (restype, argtypes); every symbol include/spectra_hip.h declares
SIGNATURES = {
    "spectra_version": (c_char_p, []),
    "spectra_last_error": (c_char_p, []),
    "spectra_w4a16_gemv": (c_int32, [ctypes.POINTER(QWeight), c_void_p, c_int64, c_int32, c_int32,
                                     c_void_p, c_int64, c_void_p]),
    "spectra_w4a16_gemv_fused": (c_int32, [ctypes.POINTER(QWeight), c_void_p, c_int64, c_int32, c_int32,
                                           ctypes.POINTER(GemvFusion), c_void_p, c_int64, c_void_p]),
    "spectra_w4a16_gemm_workspace": (c_size_t, [ctypes.POINTER(QWeight), c_int64, c_int32]),
    "spectra_w4a16_gemm": (c_int32, [ctypes.POINTER(QWeight), c_void_p, c_int64, c_int64, c_int32,
                                     c_void_p, c_int64, c_void_p, c_size_t, c_void_p]),
    "spectra_w4a16_linear": (c_int32, [ctypes.POINTER(QWeight), c_void_p, c_int64, c_int64, c_int32,
                                       c_void_p, c_int64, c_void_p, c_size_t, c_void_p]),
    "spectra_w4a16_linear_noalloc": (c_int32, [ctypes.POINTER(QWeight), c_void_p, c_int64, c_int64, c_int32,
                                               c_void_p, c_int64, c_void_p]),
    "spectra_w4_dequant": (c_int32, [ctypes.POINTER(QWeight), c_void_p, c_int64, c_int32, c_void_p]),
    "spectra_quantize_group32": (c_int32, [c_void_p, c_int64, c_int32, c_int64, c_int64, c_int32, c_void_p,
                                           c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spectra_quantize_nf4": (c_int32, [c_void_p, c_int64, c_int32, c_int64, c_int64, c_int32, c_int32, c_int32,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spectra_fwht_rows": (c_int32, [c_void_p, c_int64, c_int32, c_int64, c_int64, c_int32, c_void_p, c_int64,
                                    c_int32, c_void_p]),
    "spectra_w4_embedding": (c_int32, [ctypes.POINTER(QWeight), c_void_p, c_int64, c_void_p, c_int64, c_int32,
                                       c_void_p]),
    "spectra_outlier_columns_workspace": (c_size_t, [c_int64]),
    "spectra_outlier_columns": (c_int32, [c_void_p, c_int64, c_int32, c_int64, c_int64, c_void_p, ctypes.c_double,
                                          c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "spectra_rmsnorm": (c_int32, [c_void_p, c_void_p, c_void_p, ctypes.c_float, c_int64, c_int64, c_void_p,
                                  c_void_p]),
    "spectra_rope_append": (c_int32, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_int32, c_int32,
                                      c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spectra_attend_spans": (c_int32, [c_int32]),
    "spectra_attend_workspace": (c_size_t, [c_int32, c_int32, c_int32]),
    "spectra_attend_decode": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32,
                                        c_void_p, c_void_p, c_void_p, c_size_t, c_void_p, c_void_p]),
    "spectra_silu_mul": (c_int32, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p]),
    "spectra_greedy_next": (c_int32, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "spectra_greedy_finish": (c_int32, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "spectra_kv4_quantize": (c_int32, [c_void_p, c_int64, c_int64, c_int32, c_int64, c_int32, c_void_p, c_void_p,
                                       c_void_p, c_int64, c_void_p]),
    "spectra_kv4_dequantize": (c_int32, [c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p]),
    "spectra_attend_decode_q4": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32,
                                           c_int32] + [c_void_p] * 8 + [c_void_p, c_size_t, c_void_p, c_void_p]),
    "spectra_measure_empty": (c_int32, [c_int32, c_int32, c_void_p]),
    "spectra_measure_read": (c_int32, [c_void_p, c_size_t, c_int32, c_int32, c_void_p, c_void_p]),
}

_lock = threading.Lock()
_lib = None


class SpectraError(RuntimeError):
    """A C-ABI call returned a failure status."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} failed ({status}): {msg}")
        self.status = status


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library once; raise (never fall back) when it is unavailable."""
    global _lib
    if _lib is not None:  # loaded: no lock on the per-call path
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built; run `python -m spectra_amd._build` (hipcc, gfx950)")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


_ops_loaded = False


def load_torch_ops(path: str = TORCH_OPS_PATH):
    """Register torch.ops.spectra_hip (the operator library built beside libspectra_hip.so)
    once and return the namespace; raise (never fall back) when it is unavailable."""
    global _ops_loaded
    import torch

    if not _ops_loaded:
        with _lock:
            if not _ops_loaded:
                if not os.path.exists(path):
                    raise RuntimeError(f"{path} is not built; run `python -m spectra_amd._build`")
                torch.ops.load_library(path)
                _ops_loaded = True
    return torch.ops.spectra_hip


def check(fn_name: str, status: int) -> None:
    if status != OK:
        msg = load().spectra_last_error().decode(errors="replace")
        if status == ERR_INVALID:
            raise ValueError(f"{fn_name}: {msg}")
        raise SpectraError(fn_name, status, msg)
