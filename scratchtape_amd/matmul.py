"""`gpu_step::matmul` on MI355X: MatRef, Epilogue, matmul / matmul_f32 / matmul_with.

Mirrors gpu_step/matmul.rs:26-112: same type and argument meaning, buffers are
torch device tensors (float32, contiguous) standing in for cubecl Handles, and
offsets/strides are in elements of the whole buffer.  A failed call raises
ScratchtapeError with the message the reference would panic with.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field, replace
from typing import Optional, Tuple

import torch

from . import _lib


def _ptr(t: torch.Tensor) -> int:
    if not isinstance(t, torch.Tensor):
        raise TypeError("buffers are torch tensors")
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise ValueError("buffers are contiguous float32 tensors")
    if not t.is_cuda:
        raise ValueError("buffers live on the GPU")
    return t.data_ptr()


def _stream(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


@dataclass(frozen=True)
class MatRef:
    """A matrix inside a device buffer (matmul.rs:26-40).

    Matrix z starts at off + (z // group)*stride + (z % group)*inner; its stored
    rows are `ld` apart (0: packed); `trans`: a logical [r, c] stored as [c, r].
    """
    h: torch.Tensor
    off: int = 0
    stride: int = 0
    trans: bool = False
    ld: int = 0
    group: int = 1
    inner: int = 0

    @staticmethod
    def new(h: torch.Tensor) -> "MatRef":
        """The whole buffer from 0, one batch, not transposed (matmul.rs:44-46)."""
        return MatRef(h)

    @staticmethod
    def heads(h: torch.Tensor, col0: int, cols: int, t: int, heads: int, width: int) -> "MatRef":
        """Attention heads in place (matmul.rs:48-54): matrix z = b*heads + h is rows
        b*t .. b*t + t, columns col0 + h*width .. + width of a row-major [B*t, cols] buffer."""
        return MatRef(h, off=col0, stride=t * cols, ld=cols, group=heads, inner=width)

    def with_(self, **kw) -> "MatRef":
        return replace(self, **kw)

    def _c(self) -> _lib.StMatRef:
        return _lib.StMatRef(_ptr(self.h), self.off, self.stride, int(bool(self.trans)), 0, self.ld, self.group,
                             self.inner)


@dataclass
class Epilogue:
    """matmul.rs:62-79.  bias/mask/residual are (buffer, offset) pairs; col_sum is
    (offset, stride) into out's buffer (always +=)."""
    bias: Optional[Tuple[torch.Tensor, int]] = None
    bias_stride: int = 0
    relu: bool = False
    mask: Optional[Tuple[torch.Tensor, int]] = None
    residual: Optional[Tuple[torch.Tensor, int]] = None
    accumulate: bool = False
    col_sum: Optional[Tuple[int, int]] = None

    def _c(self) -> _lib.StEpilogue:
        e = _lib.StEpilogue()
        if self.bias is not None:
            e.bias, e.bias_off = _ptr(self.bias[0]), self.bias[1]
        e.bias_stride = self.bias_stride
        if self.mask is not None:
            e.mask, e.mask_off = _ptr(self.mask[0]), self.mask[1]
        if self.residual is not None:
            e.residual, e.residual_off = _ptr(self.residual[0]), self.residual[1]
        e.relu = int(self.relu)
        e.accumulate = int(self.accumulate)
        if self.col_sum is not None:
            e.has_col_sum = 1
            e.col_sum_off, e.col_sum_stride = self.col_sum
        return e


def _call(name, a: MatRef, b: MatRef, out: MatRef, batch, m, k, n, epi, *extra, stream=None):
    epi = epi or Epilogue()
    ca, cb, co, ce = a._c(), b._c(), out._c(), epi._c()
    _lib.call(name, ctypes.byref(ca), ctypes.byref(cb), ctypes.byref(co), batch, m, k, n, ctypes.byref(ce), *extra,
              _stream(stream))


def matmul(a: MatRef, b: MatRef, out: MatRef, batch: int, m: int, k: int, n: int,
           epi: Optional[Epilogue] = None, stream=None) -> None:
    """out[z] (+)= epi(a[z] @ b[z]) (matmul.rs:86); f16-in/f32-acc when enabled and the shape tiles."""
    _call("st_matmul", a, b, out, batch, m, k, n, epi, stream=stream)


def matmul_f32(a: MatRef, b: MatRef, out: MatRef, batch: int, m: int, k: int, n: int,
               epi: Optional[Epilogue] = None, stream=None) -> None:
    """`matmul` always in f32 (matmul.rs:93), the reference's attention route."""
    _call("st_matmul_f32", a, b, out, batch, m, k, n, epi, stream=stream)


def matmul_with(a: MatRef, b: MatRef, out: MatRef, batch: int, m: int, k: int, n: int,
                epi: Optional[Epilogue], use_f16: bool, stream=None) -> None:
    """`matmul` with the f16 route chosen by the caller (matmul.rs:106)."""
    _call("st_matmul_with", a, b, out, batch, m, k, n, epi, int(bool(use_f16)), stream=stream)


def matmul_grouped(calls, stream=None, noalloc: bool = False) -> None:
    """Several independent `matmul_with` calls in one submission (st_matmul_grouped).

    `calls` holds (a, b, out, batch, m, k, n, epi, use_f16) tuples, the arguments
    of matmul_with, e.g. a Linear backward's dW and dx (gpu_step/tape.rs:324-347).
    No call may read or write memory that another one writes.  noalloc: the
    same through st_matmul_grouped_noalloc (split-k partials in the library's
    fixed per-device scratch; no device allocation)."""
    calls = list(calls)
    arr = (_lib.StGemm * max(1, len(calls)))()
    for i, (a, b, out, batch, m, k, n, epi, use_f16) in enumerate(calls):
        arr[i] = _lib.StGemm(a._c(), b._c(), out._c(), (epi or Epilogue())._c(), batch, m, k, n, int(bool(use_f16)), 0)
    _lib.call("st_matmul_grouped_noalloc" if noalloc else "st_matmul_grouped", arr, len(calls), _stream(stream))


def f16_enabled() -> bool:
    """matmul.rs:97-102: on unless TRAIN_F16=0."""
    return bool(_lib.lib().st_f16_enabled())


def f16_route(m: int, k: int, n: int, col_sum: bool = False, b_trans: bool = False) -> bool:
    """Whether a shape takes the f16 route (matmul.rs:108-112, 524-534)."""
    return not (col_sum and b_trans) and k > 0 and k % 32 == 0 and m % 64 == 0 and n % 32 == 0


def sync(stream=None) -> None:
    """st_sync: waits for `stream`, then raises ScratchtapeError if a grouped f16 GEMM's bounded slot wait gave up
    since the last check (its outputs are not valid)."""
    _lib.call("st_sync", _stream(stream))


def set_wait_limit(polls: int) -> None:
    """st_set_wait_limit: polls before a slot wait of the grouped f16 kernel gives up (negative: the default)."""
    _lib.call("st_set_wait_limit", int(polls))
