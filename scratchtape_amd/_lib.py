"""ctypes binding of libscratchtape_hip.so (the C ABI in include/scratchtape_hip.h).

The library is loaded from this package's directory.  There is no fallback: if
it is missing or fails to load, every entry point raises, so no result ever
comes from anything but the HIP kernels.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libscratchtape_hip.so")

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_f32 = ctypes.c_float
_vp = ctypes.c_void_p

ST_OK = 0
ST_ERR_INVALID = -1
ST_ERR_HIP = -2
ST_ERR_OOM = -3
ST_ERR_NO_DEVICE = -4


class ScratchtapeError(RuntimeError):
    """A failed call; `status` is the st_status code, the message is st_last_error()."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class StMatRef(ctypes.Structure):
    _fields_ = [("p", _vp), ("off", _i64), ("stride", _i64), ("trans", _i32), ("reserved", _i32),
                ("ld", _i64), ("group", _i64), ("inner", _i64)]


class StEpilogue(ctypes.Structure):
    _fields_ = [("bias", _vp), ("bias_off", _i64), ("bias_stride", _i64), ("mask", _vp), ("mask_off", _i64),
                ("residual", _vp), ("residual_off", _i64), ("relu", _i32), ("accumulate", _i32),
                ("has_col_sum", _i32), ("reserved", _i32), ("col_sum_off", _i64), ("col_sum_stride", _i64)]


class StGemm(ctypes.Structure):
    _fields_ = [("a", StMatRef), ("b", StMatRef), ("out", StMatRef), ("epi", StEpilogue), ("batch", _i64),
                ("m", _i64), ("k", _i64), ("n", _i64), ("use_f16", _i32), ("reserved", _i32)]


_R = ctypes.POINTER(StMatRef)
_E = ctypes.POINTER(StEpilogue)

# name -> argtypes (restype st_status unless listed in _RESTYPES)
SIGNATURES = {
    "st_matmul": [_R, _R, _R, _i64, _i64, _i64, _i64, _E, _vp],
    "st_matmul_f32": [_R, _R, _R, _i64, _i64, _i64, _i64, _E, _vp],
    "st_matmul_with": [_R, _R, _R, _i64, _i64, _i64, _i64, _E, _i32, _vp],
    "st_matmul_grouped": [ctypes.POINTER(StGemm), _i64, _vp],
    "st_matmul_grouped_noalloc": [ctypes.POINTER(StGemm), _i64, _vp],
    "st_f16_enabled": [],
    "st_ndarray_matmul": [_vp, _vp, _vp, _i64, _i64, _i64],
    "st_softmax": [_vp, _vp, _i64, _i64, _i64, _f32, _i32, _i32, _vp],
    "st_softmax_backward": [_vp, _vp, _vp, _i64, _i64, _f32, _vp],
    "st_layer_norm": [_vp, _i64, _i64, _vp, _i64, _f32, _i64, _i64, _vp, _vp, _vp, _vp],
    "st_layer_norm_backward": [_vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i32, _i64, _i64, _vp],
    "st_attention_fused_fwd": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _i32, _vp],
    "st_attention_fused_bwd": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _vp],
    "st_knn_quantize_2bit": [_vp, _i64, _i64, _vp, _vp, _vp],
    "st_knn_search_ivf_2bit": [_vp, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp],
    "st_knn_key_norms_2bit": [_vp, _vp, _i64, _i64, _vp, _vp],
    "st_knn_set_scan_order": [_i32],
    "st_knn_search_masked_2bit": [_vp, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp],
    "st_knn_synth_store_2bit": [_u64, _i64, _i64, _i64, _vp, _vp, _vp],
    "st_knn_synth_keys_f32": [_u64, _i64, _i64, _i64, _vp, _vp],
    "st_knn_centroid_digit_bytes": [_i64, _i64],
    "st_knn_centroids_prep": [_vp, _i64, _i64, _vp, _vp, _vp, _vp],
    "st_knn_probe": [_vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _vp, _vp],
    "st_device_info": [_vp, _vp, _vp, _vp],
    "st_peak_mfma": [_i32, _i64, _i32, _vp, _vp],
    "st_peak_read": [_vp, _i64, _i32, _vp, _vp],
    "st_lane_selftest": [_vp, _vp],
    "st_last_error": [],
    "st_sync": [_vp],
    "st_set_wait_limit": [_i64],
    "st_scratch_release": [],
    "st_version": [],
}
_RESTYPES = {"st_last_error": ctypes.c_char_p, "st_version": ctypes.c_char_p, "st_f16_enabled": _i32,
             "st_knn_centroid_digit_bytes": _i64}

_lib = None


def lib():
    """The loaded library (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ScratchtapeError(ST_ERR_NO_DEVICE,
                                   f"{LIB_PATH} is not built; run `python -m scratchtape_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, _i32)
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != ST_OK:
        msg = lib().st_last_error().decode(errors="replace")
        raise ScratchtapeError(status, msg or f"status {status}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
