"""`NdArray::matmul` drop-in (src/tensor.rs:241-276) on host arrays.

The product runs on the GPU in f32 (st_ndarray_matmul: host buffers are copied
in and out inside the call).  Shapes are checked as the reference asserts them.
"""
from __future__ import annotations

import numpy as np

from . import _lib


def ndarray_matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    if a.ndim != 2:
        raise ValueError(f"matmul lhs must be 2D, got {list(a.shape)}")
    if b.ndim != 2:
        raise ValueError(f"matmul rhs must be 2D, got {list(b.shape)}")
    (m, k), (k2, n) = a.shape, b.shape
    if k != k2:
        raise ValueError(f"matmul inner dims must match: {list(a.shape)} vs {list(b.shape)}")
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty((m, n), np.float32)
    _lib.call("st_ndarray_matmul", a.ctypes.data, b.ctypes.data, out.ctypes.data, m, k, n)
    return out
