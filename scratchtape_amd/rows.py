"""Row kernels on MI355X: causal softmax and its backward (gpu_step/rows.rs:101-123),
LayerNorm forward and backward (gpu_step/rows.rs:60-99)."""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .matmul import _ptr, _stream


def _check_rows_out(out: torch.Tensor | None, n: int, device, name: str) -> None:
    """A caller-supplied output must hold every element the kernel writes (rows x n floats) on the input's
    device."""
    if out is None:
        return
    if out.numel() < n:
        raise ValueError(f"{name}: out holds {out.numel()} elements, the call writes {n}")
    if out.device != device:
        raise ValueError(f"{name}: out is on {out.device}, the input on {device}")


def softmax(x: torch.Tensor, rows: int, n: int, t: int, scale: float, causal: bool, one: bool,
            out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Row-wise softmax of scale*x over x [rows, n] (rows.rs:101-112); returns y."""
    _check_rows_out(out, rows * n, x.device, "softmax")
    y = out if out is not None else torch.empty(rows * n, dtype=torch.float32, device=x.device)
    _lib.call("st_softmax", _ptr(x), _ptr(y), rows, n, t, float(scale), int(causal), int(one), _stream(stream))
    return y


def softmax_backward(dy: torch.Tensor, y: torch.Tensor, rows: int, n: int, scale: float,
                     out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """dx = scale * y * (dy - sum(dy * y)) per row (rows.rs:114-123); returns dx."""
    _check_rows_out(out, rows * n, y.device, "softmax_backward")
    dx = out if out is not None else torch.empty(rows * n, dtype=torch.float32, device=y.device)
    _lib.call("st_softmax_backward", _ptr(dy), _ptr(y), _ptr(dx), rows, n, float(scale), _stream(stream))
    return dx


@dataclass
class LnOut:
    """What LayerNorm's backward needs from its forward (rows.rs:52-58)."""
    y: torch.Tensor
    mean: torch.Tensor
    rstd: torch.Tensor


def layer_norm(x: torch.Tensor, rows: int, d: int, params: torch.Tensor, off: int, eps: float = 1e-5,
               models: int = 1, model_stride: int = 0, stream=None) -> LnOut:
    """y = (x - mean) / sqrt(var + eps) * gamma + beta per row (rows.rs:65); gamma, beta at params[off..]."""
    dev = x.device
    out = LnOut(torch.empty(rows * d, dtype=torch.float32, device=dev), torch.empty(rows, dtype=torch.float32, device=dev),
                torch.empty(rows, dtype=torch.float32, device=dev))
    _lib.call("st_layer_norm", _ptr(x), rows, d, _ptr(params), off, float(eps), models, model_stride, _ptr(out.y),
              _ptr(out.mean), _ptr(out.rstd), _stream(stream))
    return out


def layer_norm_backward(dy: torch.Tensor, x: torch.Tensor, fwd: LnOut, rows: int, d: int, params: torch.Tensor,
                        grads: torch.Tensor, off: int, dx: torch.Tensor, accumulate: bool, models: int = 1,
                        model_stride: int = 0, stream=None) -> None:
    """dx (+)= LayerNorm's input gradient; gamma / beta gradients accumulate into grads at off (rows.rs:90)."""
    _lib.call("st_layer_norm_backward", _ptr(dy), _ptr(x), _ptr(fwd.mean), _ptr(fwd.rstd), rows, d, _ptr(params),
              _ptr(grads), off, _ptr(dx), int(accumulate), models, model_stride, _stream(stream))
