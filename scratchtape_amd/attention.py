"""Batched causal attention forward and backward as the device tape runs it.

The call sequence of DeviceTape::batched_matmul / backward and the softmax
between them (gpu_step/tape.rs:196-212, 349-372, 475-491; rows.rs:101-123):
Q, K, V are head views of a fused [B*T, 3D] buffer, the scores S and
probabilities P are stacked [B*H*T, T], the context is written into the merged
[B*T, D] layout.  Every product goes through the GEMM of this package and the
softmax through its row kernels; `use_f16` picks the f16-in/f32-acc route for
the six products (the reference keeps them f32: matmul.rs:90-95).

`fused_forward` / `fused_backward` compute the same attention in two launches
that never write S or P (the reference's next step, docs/tiers_design.md:891-893):
the forward keeps each row's log-sum-exp, from which the backward recomputes P.
They run the f16-in/f32-acc route for head_dim 64 and sequence lengths that are
multiples of 32 up to 256.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib, rows
from .matmul import Epilogue, MatRef, _stream, matmul_with


@dataclass
class AttnBuffers:
    s: torch.Tensor     # [B*H*T, T] scores
    p: torch.Tensor     # [B*H*T, T] probabilities
    ctx: torch.Tensor   # [B*T, D] context
    dp: torch.Tensor    # [B*H*T, T]
    ds: torch.Tensor    # [B*H*T, T]
    dqkv: torch.Tensor  # [B*T, 3D] gradient of the fused QKV buffer

    @staticmethod
    def empty(b: int, h: int, t: int, hd: int, device) -> "AttnBuffers":
        d = h * hd
        z = lambda n: torch.zeros(n, dtype=torch.float32, device=device)
        return AttnBuffers(z(b * h * t * t), z(b * h * t * t), z(b * t * d), z(b * h * t * t), z(b * h * t * t),
                           z(b * t * 3 * d))


def forward(qkv: torch.Tensor, buf: AttnBuffers, b: int, h: int, t: int, hd: int, use_f16: bool,
            stream=None) -> None:
    d = h * hd
    batch, scale = b * h, hd ** -0.5
    stacked = MatRef(buf.s, stride=t * t)
    matmul_with(MatRef.heads(qkv, 0, 3 * d, t, h, hd), MatRef.heads(qkv, d, 3 * d, t, h, hd).with_(trans=True),
                stacked, batch, t, hd, t, None, use_f16, stream=stream)
    rows.softmax(buf.s, batch * t, t, t, scale, True, False, out=buf.p, stream=stream)
    matmul_with(MatRef(buf.p, stride=t * t), MatRef.heads(qkv, 2 * d, 3 * d, t, h, hd),
                MatRef.heads(buf.ctx, 0, d, t, h, hd), batch, t, t, hd, None, use_f16, stream=stream)


def backward(qkv: torch.Tensor, dctx: torch.Tensor, buf: AttnBuffers, b: int, h: int, t: int, hd: int,
             use_f16: bool, stream=None) -> None:
    """dV = Pᵀ dO, dP = dO Vᵀ, dS = softmax backward, dQ = dS K, dK = dSᵀ Q, written into buf.dqkv."""
    d = h * hd
    batch, scale = b * h, hd ** -0.5
    p = MatRef(buf.p, stride=t * t)
    do = MatRef.heads(dctx, 0, d, t, h, hd)
    v = MatRef.heads(qkv, 2 * d, 3 * d, t, h, hd)
    # c = p v: dp = dc vᵀ, dv = pᵀ dc
    matmul_with(do, v.with_(trans=True), MatRef(buf.dp, stride=t * t), batch, t, hd, t, None, use_f16,
                stream=stream)
    matmul_with(p.with_(trans=True), do, MatRef.heads(buf.dqkv, 2 * d, 3 * d, t, h, hd), batch, t, t, hd, None,
                use_f16, stream=stream)
    rows.softmax_backward(buf.dp, buf.p, batch * t, t, scale, out=buf.ds, stream=stream)
    # s = q kᵀ: dq = ds k, dk = dsᵀ q
    ds = MatRef(buf.ds, stride=t * t)
    matmul_with(ds, MatRef.heads(qkv, d, 3 * d, t, h, hd), MatRef.heads(buf.dqkv, 0, 3 * d, t, h, hd), batch, t, t,
                hd, None, use_f16, stream=stream)
    matmul_with(ds.with_(trans=True), MatRef.heads(qkv, 0, 3 * d, t, h, hd),
                MatRef.heads(buf.dqkv, d, 3 * d, t, h, hd), batch, t, t, hd, None, use_f16, stream=stream)


def step(qkv: torch.Tensor, dctx: torch.Tensor, buf: AttnBuffers, b: int, h: int, t: int, hd: int,
         use_f16: bool, stream: Optional[object] = None) -> None:
    forward(qkv, buf, b, h, t, hd, use_f16, stream)
    backward(qkv, dctx, buf, b, h, t, hd, use_f16, stream)


@dataclass
class FusedBuffers:
    ctx: torch.Tensor   # [B*T, D] context
    lse: torch.Tensor   # [B*H*T] log-sum-exp of each score row (kept for the backward)
    dqkv: torch.Tensor  # [B*T, 3D] gradient of the fused QKV buffer

    @staticmethod
    def empty(b: int, h: int, t: int, hd: int, device) -> "FusedBuffers":
        d = h * hd
        z = lambda n: torch.zeros(n, dtype=torch.float32, device=device)
        return FusedBuffers(z(b * t * d), z(b * h * t), z(b * t * 3 * d))


def _f32(t: torch.Tensor, what: str) -> int:
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous():
        raise ValueError(f"{what} must be a contiguous float32 GPU tensor")
    return t.data_ptr()


def fused_forward(qkv: torch.Tensor, buf: FusedBuffers, b: int, h: int, t: int, hd: int, one: bool = False,
                  stream=None) -> None:
    """O = softmax(hd^-1/2 Q K^T, causal) V into buf.ctx, row log-sum-exp into buf.lse."""
    _lib.call("st_attention_fused_fwd", _f32(qkv, "qkv"), _f32(buf.ctx, "ctx"), _f32(buf.lse, "lse"), b, h, t, hd,
              hd ** -0.5, int(one), _stream(stream))


def fused_backward(qkv: torch.Tensor, dctx: torch.Tensor, buf: FusedBuffers, b: int, h: int, t: int, hd: int,
                   stream=None) -> None:
    """dQ, dK, dV of the fused forward for the upstream gradient dctx, into buf.dqkv."""
    _lib.call("st_attention_fused_bwd", _f32(qkv, "qkv"), _f32(buf.ctx, "ctx"), _f32(dctx, "dctx"),
              _f32(buf.lse, "lse"), _f32(buf.dqkv, "dqkv"), b, h, t, hd, hd ** -0.5, _stream(stream))


def fused_step(qkv: torch.Tensor, dctx: torch.Tensor, buf: FusedBuffers, b: int, h: int, t: int, hd: int,
               one: bool = False, stream: Optional[object] = None) -> None:
    fused_forward(qkv, buf, b, h, t, hd, one, stream)
    fused_backward(qkv, dctx, buf, b, h, t, hd, stream)
