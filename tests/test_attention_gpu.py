"""Batched causal attention (B=32 windows x H=4 heads, T=128, head 64) forward and
backward on the GPU against the CPU oracle's per-chunk loop (tape.rs:73-112).

Tolerances (scale-relative): f32 route 1e-5 on P and O, 1e-4 on the gradients
(the softmax backward subtracts nearly equal terms); f16-in route 2e-3 against
the oracle run on f16-rounded Q, K, V (the BJ attention contract).  Softmax
kernels alone: forward 1e-5, backward 1e-4 (rows.rs:497-500).
"""
import random

import numpy as np
import pytest
import torch

import oracle
from scratchtape_amd import attention, rows

pytestmark = pytest.mark.gpu

B, H, T, HD = 32, 4, 128, 64
D = H * HD


def rel_err(got, want):
    return float(np.max(np.abs(got - want))) / max(float(np.max(np.abs(want))), 1e-30)


def split_heads(x, col0):
    """[B*T, cols] buffer -> chunk-major [B*H, T, HD] heads starting at column col0."""
    cols = x.shape[1]
    return x.reshape(B, T, cols)[:, :, col0:col0 + D].reshape(B, T, H, HD).transpose(0, 2, 1, 3).reshape(B * H, T, HD)


@pytest.mark.parametrize("use_f16", [False, True])
def test_attention_step_matches_oracle(dev, use_f16):
    rng = oracle.Rng(17)
    qkv = rng.gaussian(B * T * 3 * D).reshape(B * T, 3 * D)
    dctx = rng.gaussian(B * T * D).reshape(B * T, D)
    if use_f16:
        qkv = oracle.round_f16(qkv)  # f16 Q, K, V
    qkv_d = torch.from_numpy(qkv).to(dev).reshape(-1)
    dctx_d = torch.from_numpy(dctx).to(dev).reshape(-1)
    buf = attention.AttnBuffers.empty(B, H, T, HD, dev)
    attention.step(qkv_d, dctx_d, buf, B, H, T, HD, use_f16)
    torch.cuda.synchronize()

    q, k, v = split_heads(qkv, 0), split_heads(qkv, D), split_heads(qkv, 2 * D)
    do = split_heads(dctx, 0)
    p, o, dq, dk, dv = oracle.attention_fwd_bwd(q, k, v, do, B * H, T, HD, HD ** -0.5)
    dqkv = buf.dqkv.cpu().numpy().reshape(B * T, 3 * D)
    got = {
        "P": buf.p.cpu().numpy(),
        "O": split_heads(buf.ctx.cpu().numpy().reshape(B * T, D), 0).reshape(-1),
        "dQ": split_heads(dqkv, 0).reshape(-1),
        "dK": split_heads(dqkv, D).reshape(-1),
        "dV": split_heads(dqkv, 2 * D).reshape(-1),
    }
    want = {"P": p, "O": o, "dQ": dq, "dK": dk, "dV": dv}
    for name in want:
        e = rel_err(got[name], want[name])
        tol = 2e-3 if use_f16 else (1e-5 if name in ("P", "O") else 1e-4)
        assert e <= tol, f"{name}: {e} (f16 {use_f16})"
    # masked entries are exactly zero
    P = got["P"].reshape(B * H, T, T)
    assert np.all(P[:, np.triu_indices(T, 1)[0], np.triu_indices(T, 1)[1]] == 0.0)


@pytest.mark.parametrize("one,amp,n,t", [(False, 1.0, 128, 128), (True, 1.0, 128, 128), (True, 40.0, 64, 64),
                                          (False, 3.0, 200, 50), (False, 1.0, 7, 7)])
def test_softmax_kernels_match_oracle(dev, one, amp, n, t):
    rows_ = 3 * n
    rng = oracle.Rng(3)
    x = rng.gaussian(rows_ * n) * np.float32(amp)
    dy = rng.gaussian(rows_ * n)
    scale = 0.125
    xd = torch.from_numpy(x).to(dev)
    y = rows.softmax(xd, rows_, n, t, scale, True, one)
    dx = rows.softmax_backward(torch.from_numpy(dy).to(dev), y, rows_, n, scale)
    want_y = oracle.softmax(x, rows_, n, t, scale, True, one)
    want_dx = oracle.softmax_backward(dy, want_y, rows_, n, scale)
    assert rel_err(y.cpu().numpy(), want_y) <= 1e-5
    assert rel_err(dx.cpu().numpy(), want_dx) <= 1e-4
    yy = y.cpu().numpy().reshape(rows_, n)
    for r in range(rows_):
        assert np.all(yy[r, (r % t) + 1:] == 0.0)


# --------------------------------------------------------------------------- fused attention


def fused_case(dev, b, h, t, one, seed):
    d = h * HD
    rng = oracle.Rng(seed)
    qkv = oracle.round_f16(rng.gaussian(b * t * 3 * d).reshape(b * t, 3 * d))  # f16 Q, K, V
    dctx = rng.gaussian(b * t * d).reshape(b * t, d)
    buf = attention.FusedBuffers.empty(b, h, t, HD, dev)
    attention.fused_step(torch.from_numpy(qkv).to(dev).reshape(-1), torch.from_numpy(dctx).to(dev).reshape(-1), buf,
                         b, h, t, HD, one)
    torch.cuda.synchronize()
    heads = lambda x, c0, cols: x.reshape(b, t, cols)[:, :, c0:c0 + d].reshape(b, t, h, HD).transpose(0, 2, 1, 3) \
        .reshape(b * h, t, HD)
    q, k, v, do = heads(qkv, 0, 3 * d), heads(qkv, d, 3 * d), heads(qkv, 2 * d, 3 * d), heads(dctx, 0, d)
    _, o, dq, dk, dv = oracle.attention_fwd_bwd(q, k, v, do, b * h, t, HD, HD ** -0.5, one)
    dqkv = buf.dqkv.cpu().numpy().reshape(b * t, 3 * d)
    got = {"O": heads(buf.ctx.cpu().numpy().reshape(b * t, d), 0, d), "dQ": heads(dqkv, 0, 3 * d),
           "dK": heads(dqkv, d, 3 * d), "dV": heads(dqkv, 2 * d, 3 * d)}
    want = {"O": o, "dQ": dq, "dK": dk, "dV": dv}
    for name in want:
        e = rel_err(got[name].reshape(-1), want[name].reshape(-1))
        assert e <= 2e-3, f"{name}: {e} (b {b} h {h} t {t} one {one})"
    # The saved row statistic is log(sum(exp(scale S))) over the causal row (plus softmax1's phantom).
    S = np.einsum("zic,zjc->zij", q.astype(np.float64), k.astype(np.float64)) * HD ** -0.5
    S = np.where(np.tril(np.ones((t, t), bool))[None], S, -np.inf)
    mx = S.max(-1)
    if one:
        mx = np.maximum(mx, 0.0)
    lse = mx + np.log(np.exp(S - mx[..., None]).sum(-1) + (np.exp(-mx) if one else 0.0))
    assert np.max(np.abs(buf.lse.cpu().numpy().reshape(b * h, t) - lse)) <= 2e-3 * max(1.0, np.max(np.abs(lse)))
    return buf


def test_fused_attention_at_the_configured_shape(dev):
    fused_case(dev, B, H, T, False, 17)


@pytest.mark.parametrize("b,h,t,one", [(2, 3, 32, False), (3, 1, 64, True), (2, 2, 96, False), (1, 2, 160, False),
                                        (2, 1, 256, True), (1, 5, 128, True)])
def test_fused_attention_shapes_and_softmax1(dev, b, h, t, one):
    fused_case(dev, b, h, t, one, 100 + t)


def test_fused_attention_agrees_with_the_unfused_f16_route(dev):
    rng = oracle.Rng(23)
    qkv = torch.from_numpy(oracle.round_f16(rng.gaussian(B * T * 3 * D))).to(dev)
    dctx = torch.from_numpy(rng.gaussian(B * T * D)).to(dev)
    ub = attention.AttnBuffers.empty(B, H, T, HD, dev)
    attention.step(qkv, dctx, ub, B, H, T, HD, True)
    fb = attention.FusedBuffers.empty(B, H, T, HD, dev)
    attention.fused_step(qkv, dctx, fb, B, H, T, HD)
    torch.cuda.synchronize()
    assert rel_err(fb.ctx.cpu().numpy(), ub.ctx.cpu().numpy()) <= 2e-3
    assert rel_err(fb.dqkv.cpu().numpy(), ub.dqkv.cpu().numpy()) <= 4e-3


def test_fused_attention_random_shapes(dev):
    # Seeded random batches, head counts, every T = 32 .. 256 step 32 among them, softmax1 or not.
    rnd = random.Random(23)
    for i, t in enumerate(rnd.sample(range(32, 257, 32), 8)):
        fused_case(dev, rnd.randint(1, 3), rnd.randint(1, 4), t, rnd.random() < 0.5, 300 + i)
