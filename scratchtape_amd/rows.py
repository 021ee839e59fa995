"""Causal softmax and its backward (gpu_step/rows.rs:101-123) on MI355X."""
from __future__ import annotations

import torch

from . import _lib
from .matmul import _ptr, _stream


def softmax(x: torch.Tensor, rows: int, n: int, t: int, scale: float, causal: bool, one: bool,
            out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Row-wise softmax of scale*x over x [rows, n] (rows.rs:101-112); returns y."""
    y = out if out is not None else torch.empty(rows * n, dtype=torch.float32, device=x.device)
    _lib.call("st_softmax", _ptr(x), _ptr(y), rows, n, t, float(scale), int(causal), int(one), _stream(stream))
    return y


def softmax_backward(dy: torch.Tensor, y: torch.Tensor, rows: int, n: int, scale: float,
                     out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """dx = scale * y * (dy - sum(dy * y)) per row (rows.rs:114-123); returns dx."""
    dx = out if out is not None else torch.empty(rows * n, dtype=torch.float32, device=y.device)
    _lib.call("st_softmax_backward", _ptr(dy), _ptr(y), _ptr(dx), rows, n, float(scale), _stream(stream))
    return dx
