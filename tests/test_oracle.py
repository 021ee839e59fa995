"""Pins the CPU oracle (oracle/oracle.c) before the parity tests rely on it.

Each check is chosen so that a plausible mistake in the restatement (a wrong
shift or constant, FMA contraction, a wrong index, a transposed operand, a
wrong rounding rule) fails it: published known answers, exact integer
arithmetic, independent library routines (numpy float16 / float64) and
brute force on small inputs.
"""
import math

import numpy as np
import pytest

import oracle

# --------------------------------------------------------------------------- Rng (nn.rs:8-35)


def test_xorshift64_matches_marsaglias_published_sequence():
    # G. Marsaglia, "Xorshift RNGs", J. Stat. Softw. 8(14), 2003: xor64() with
    # (13, 7, 17) from 88172645463325252 yields these first outputs.
    r = oracle.Rng(88172645463325252)
    states = []
    for _ in range(3):
        r.next_f32()
        states.append(r.state.value)
    assert states == [8748534153485358512, 3040900993826735515, 3453997556048239312]


def test_xorshift64_big_int_recurrence_for_other_seeds():
    mask = (1 << 64) - 1
    for seed in (1, 5, 42, 0xDEADBEEF, mask):
        x = seed
        r = oracle.Rng(seed)
        for _ in range(50):
            x ^= (x << 13) & mask
            x ^= x >> 7
            x ^= (x << 17) & mask
            f = r.next_f32()
            assert r.state.value == x
            # next_f32 is the f32 rounding of x / (2^64 - 1): within half an f32 ulp of the exact ratio.
            exact = x / mask
            assert abs(f - exact) <= 0.5 * np.spacing(np.float32(exact)) * 1.0001 + 1e-45


def test_next_f32_uniform_and_gaussian_moments():
    r = oracle.Rng(7)
    u = r.uniform(200_000)
    assert u.min() >= -1.0 and u.max() <= 1.0
    assert abs(u.mean()) < 0.01 and abs(u.var() - 1 / 3) < 0.01
    g = r.gaussian(200_000)
    assert abs(g.mean()) < 0.01 and abs(g.var() - 1.0) < 0.015


def test_gaussian_is_box_muller_of_the_next_two_uniforms():
    a, b = oracle.Rng(99), oracle.Rng(99)
    for _ in range(500):
        u1 = max(a.next_f32(), 1e-9)
        u2 = a.next_f32()
        want = math.sqrt(-2.0 * math.log(u1)) * math.cos(2.0 * math.pi * u2)
        got = b.next_gaussian()
        assert abs(got - want) <= 2e-6 * max(1.0, abs(want))


# --------------------------------------------------------------------------- matmul (tensor.rs:241-276)


def test_matmul_known_answer_from_gpu_rs():
    # gpu.rs:176-185
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    np.testing.assert_array_equal(oracle.matmul(a, b), [[58, 64], [139, 154]])


@pytest.mark.parametrize("m,k,n", [(37, 53, 29), (130, 70, 65), (1, 200, 3), (64, 64, 64), (65, 129, 7)])
def test_matmul_integer_inputs_are_exact(m, k, n):
    rng = np.random.default_rng(m * 1000 + k)
    a = rng.integers(-8, 9, (m, k))
    b = rng.integers(-8, 9, (k, n))
    np.testing.assert_array_equal(oracle.matmul(a.astype(np.float32), b.astype(np.float32)), (a @ b).astype(np.float32))


def test_matmul_identity_and_permutation():
    rng = np.random.default_rng(3)
    a = rng.standard_normal((40, 70)).astype(np.float32)
    np.testing.assert_array_equal(oracle.matmul(a, np.eye(70, dtype=np.float32)), a)
    perm = rng.permutation(70)
    p = np.eye(70, dtype=np.float32)[perm].T  # a @ p permutes the columns
    np.testing.assert_array_equal(oracle.matmul(a, p), a[:, perm])
    np.testing.assert_array_equal(oracle.matmul(np.eye(40, dtype=np.float32), a), a)


def test_matmul_sums_p_ascending_without_fma():
    # The reference accumulates out[i,j] over p = 0..k-1 in order, rounding
    # the product and the sum separately.  An independent numpy float32
    # accumulation in that order must agree bit for bit; the fused (FMA) order
    # must not (so contraction would be caught).
    r = oracle.Rng(42)
    m, k, n = 37, 150, 29
    a = r.uniform(m * k).reshape(m, k)
    b = r.uniform(k * n).reshape(k, n)
    seq = np.zeros((m, n), np.float32)
    fused = np.zeros((m, n), np.float32)
    for p in range(k):
        seq = (seq + (a[:, p:p + 1] * b[p:p + 1, :]).astype(np.float32)).astype(np.float32)
        fused = (fused.astype(np.float64) + a[:, p:p + 1].astype(np.float64) * b[p:p + 1, :].astype(np.float64)).astype(np.float32)
    got = oracle.matmul(a, b)
    np.testing.assert_array_equal(got, seq)
    assert np.any(got != fused)
    ref64 = a.astype(np.float64) @ b.astype(np.float64)
    assert np.max(np.abs(got - ref64)) <= 1e-5 * np.max(np.abs(ref64))


def test_transpose():
    a = np.arange(35, dtype=np.float32).reshape(5, 7)
    np.testing.assert_array_equal(oracle.transpose(a), a.T)
    np.testing.assert_array_equal(oracle.transpose(oracle.transpose(a)), a)


# --------------------------------------------------------------------------- f16 rounding (half 2.7.1, RNE)


@pytest.mark.parametrize("x,bits", [
    (1.0, 0x3C00), (-2.0, 0xC000), (65504.0, 0x7BFF), (65519.99, 0x7BFF), (65520.0, 0x7C00),
    (2049.0, 0x6800), (2051.0, 0x6802), (2050.0, 0x6801), (2.0 ** -24, 0x0001), (2.0 ** -25, 0x0000),
    (3 * 2.0 ** -25, 0x0002), (2.0 ** -14, 0x0400), (0.1, 0x2E66), (-0.0, 0x8000), (1e10, 0x7C00),
    (float("inf"), 0x7C00), (-float("inf"), 0xFC00), (2.0 ** -14 - 2.0 ** -25, 0x0400), (0.333333, 0x3555),
])
def test_f16_rounding_known_answers(x, bits):
    assert oracle.f32_to_f16_bits(x) == bits


def test_f16_rounding_matches_numpy_over_all_ranges():
    rng = np.random.default_rng(0)
    mags = np.exp2(rng.uniform(-30, 17, 400_000)).astype(np.float32)
    xs = np.concatenate([mags, -mags, rng.standard_normal(100_000).astype(np.float32)])
    # exact ties of the f16 grid
    grid = np.arange(1, 2048, dtype=np.float32)
    xs = np.concatenate([xs, grid + 2048.0 + 0.5 * 0, (grid * 2 + 1) * np.float32(2.0 ** -25)]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(oracle.round_f16(xs), want)


# --------------------------------------------------------------------------- gpu_step::matmul semantics

def _np_operand(buf, off, stride, trans, ld, group, inner, z, rows, cols):
    """Logical [rows, cols] matrix z of a MatRef, by explicit numpy indexing."""
    g = max(group, 1)
    base = off + (z // g) * stride + (z % g) * inner
    if trans:
        ldv = ld or rows
        idx = base + np.arange(cols)[:, None] * ldv + np.arange(rows)[None, :]
        return buf[idx].T
    ldv = ld or cols
    idx = base + np.arange(rows)[:, None] * ldv + np.arange(cols)[None, :]
    return buf[idx]


# (batch, m, k, n, ta, tb, bias, relu, mask, res, acc): the f32 case list of matmul.rs:987-1007
CASES_F32 = [
    (1, 70, 35, 20, False, False, False, False, False, False, False),
    (1, 70, 35, 20, True, False, False, False, False, False, False),
    (1, 70, 35, 20, False, True, False, False, False, False, False),
    (1, 70, 35, 20, True, True, False, False, False, False, False),
    (3, 33, 17, 65, False, True, True, True, False, False, False),
    (3, 64, 64, 64, True, False, False, False, False, True, True),
    (1, 128, 64, 96, False, False, True, False, False, False, False),
    (2, 33, 17, 65, True, False, True, True, True, True, True),
    (64, 16, 16, 16, False, True, False, False, False, False, False),
]


@pytest.mark.parametrize("case", CASES_F32)
@pytest.mark.parametrize("f16", [False, True])
def test_gemm_semantics_exact_on_integer_data(case, f16):
    batch, m, k, n, ta, tb, has_bias, relu, has_mask, has_res, acc = case
    rng = np.random.default_rng(hash(case) % 2**32)
    ints = lambda size: rng.integers(-4, 5, size).astype(np.float32)  # exact in f16 and f32
    a_off, b_off, o_off, bias_off, m_off, r_off = 3, 5, 7, 2, 6, 1
    sa, sb, so = m * k + 1, (k * n + 2 if batch > 1 else 0), m * n + 3
    a = ints(a_off + batch * sa)
    b = ints(b_off + max(batch, 1) * max(sb, k * n))
    bias_stride = n + 1 if batch > 1 else 0
    bias = ints(bias_off + batch * (n + 1))
    res = ints(r_off + batch * so)
    mask = ints(m_off + batch * so)
    cs_off, cs_stride = o_off + batch * so + 5, n + 3
    out0 = ints(cs_off + batch * cs_stride + 2)

    want = out0.astype(np.float64).copy()
    for z in range(batch):
        A = _np_operand(a, a_off, sa, ta, 0, 1, 0, z, m, k).astype(np.int64)
        B = _np_operand(b, b_off, sb, tb, 0, 1, 0, z, k, n).astype(np.int64)
        want[cs_off + z * cs_stride: cs_off + z * cs_stride + n] += B.sum(axis=0)
        s = (A @ B).astype(np.float64)
        if has_bias:
            s += bias[bias_off + z * bias_stride: bias_off + z * bias_stride + n][None, :]
        if relu:
            s = np.maximum(s, 0)
        idx = z * so + np.arange(m)[:, None] * n + np.arange(n)[None, :]
        if has_mask:
            s = np.where(mask[m_off + idx] <= 0, 0.0, s)
        if has_res:
            s = s + res[r_off + idx]
        if acc:
            s = s + want[o_off + idx]
        want[o_off + idx] = s

    got = out0.copy()
    oracle.gemm(a, dict(off=a_off, stride=sa, trans=ta), b, dict(off=b_off, stride=sb, trans=tb), got,
                dict(off=o_off, stride=so), batch, m, k, n,
                bias=(bias, bias_off) if has_bias else None, bias_stride=bias_stride, relu=relu,
                mask=(mask, m_off) if has_mask else None, residual=(res, r_off) if has_res else None,
                accumulate=acc, col_sum=(cs_off, cs_stride), f16=f16)
    np.testing.assert_array_equal(got, want.astype(np.float32))


def test_gemm_head_views_match_split_heads_slicing():
    # Head views of matmul.rs:48-54 against explicit split-heads slicing (tape.rs:119-134): B 2, H 3, t 5, w 4.
    bsz, heads, t, w = 2, 3, 5, 4
    hw, fused = heads * w, 3 * heads * w
    rng = np.random.default_rng(9)
    qkv = rng.integers(-4, 5, bsz * t * fused).astype(np.float32)
    batch = bsz * heads
    X = qkv.reshape(bsz, t, fused)
    heads_of = lambda col0: X[:, :, col0:col0 + hw].reshape(bsz, t, heads, w).transpose(0, 2, 1, 3).reshape(batch, t, w)
    Q, K = heads_of(0).astype(np.int64), heads_of(hw).astype(np.int64)
    want = np.einsum("zic,zjc->zij", Q, K).astype(np.float32).reshape(-1)
    got = np.zeros(batch * t * t, np.float32)
    hv = lambda col0: dict(off=col0, stride=t * fused, ld=fused, group=heads, inner=w)
    oracle.gemm(qkv, hv(0), qkv, dict(hv(hw), trans=True), got, dict(stride=t * t), batch, t, w, t)
    np.testing.assert_array_equal(got, want)


# --------------------------------------------------------------------------- LayerNorm (nn.rs, rows.rs)


def _ln_params(d, off, models=1, stride=None):
    stride = stride if stride is not None else 2 * d
    flat = np.full(off + (models - 1) * stride + 2 * d + 1, 9.0, np.float32)
    for m in range(models):
        j = np.arange(d)
        flat[off + m * stride: off + m * stride + d] = 1.0 + 0.1 * ((j * 7 + m) % 5)   # gamma (rows.rs:416-417)
        flat[off + m * stride + d: off + m * stride + 2 * d] = 0.05 * ((j * 3 + m) % 4) - 0.1  # beta
    return flat, stride


@pytest.mark.parametrize("rows,d,off", [(37, 24, 5), (37, 200, 3), (203, 24, 5)])
def test_layer_norm_matches_float64_closed_form(rows, d, off):
    rng = oracle.Rng(7)
    x = rng.gaussian(rows * d).reshape(rows, d)
    r = rng.gaussian(rows * d).reshape(rows, d)
    params, _ = _ln_params(d, off)
    y, mean, rstd = oracle.layer_norm(x, rows, d, params, off, 1e-5)
    X = x.astype(np.float64)
    mu = X.mean(1, keepdims=True)
    var = ((X - mu) ** 2).mean(1, keepdims=True)
    xh = (X - mu) / np.sqrt(var + 1e-5)
    gam, bet = params[off:off + d].astype(np.float64), params[off + d:off + 2 * d].astype(np.float64)
    Y = xh * gam + bet
    assert np.max(np.abs(y.reshape(rows, d) - Y)) <= 1e-5 * np.max(np.abs(Y))
    assert np.allclose(mean, mu[:, 0], atol=1e-6) and np.allclose(rstd, 1 / np.sqrt(var[:, 0] + 1e-5), rtol=1e-5)
    # Normalised rows (gamma 1, beta 0): mean 0, biased variance var / (var + eps).
    ones = np.concatenate([np.ones(d, np.float32), np.zeros(d, np.float32)])
    y1, _, _ = oracle.layer_norm(x, rows, d, ones, 0, 1e-5)
    y1 = y1.reshape(rows, d).astype(np.float64)
    assert np.max(np.abs(y1.mean(1))) < 1e-6 and np.allclose(y1.var(1), (var / (var + 1e-5))[:, 0], rtol=1e-5)
    # Backward of sum(r * y): dx against float64 closed form and finite differences, dgamma / dbeta as column sums.
    grads = np.full(params.size, 0.5, np.float32)
    dx = oracle.layer_norm_backward(r, x, mean, rstd, rows, d, params, grads, off)
    R = r.astype(np.float64)
    g = R * gam
    DX = (g - g.mean(1, keepdims=True) - xh * (g * xh).mean(1, keepdims=True)) / np.sqrt(var + 1e-5)
    assert np.max(np.abs(dx.reshape(rows, d) - DX)) <= 1e-4 * np.max(np.abs(DX))
    assert np.allclose(grads[off:off + d], 0.5 + (R * xh).sum(0), rtol=1e-4, atol=1e-4)
    assert np.allclose(grads[off + d:off + 2 * d], 0.5 + R.sum(0), rtol=1e-4, atol=1e-4)
    assert np.all(grads[:off] == 0.5) and np.all(grads[off + 2 * d:] == 0.5)
    def loss(xx):
        X2 = xx.astype(np.float64)
        m2 = X2.mean(1, keepdims=True)
        v2 = ((X2 - m2) ** 2).mean(1, keepdims=True)
        return (R * (((X2 - m2) / np.sqrt(v2 + 1e-5)) * gam + bet)).sum()
    for (i, j) in [(0, 0), (rows // 2, d - 1), (rows - 1, 3)]:
        xp, xm = x.astype(np.float64).copy(), x.astype(np.float64).copy()
        xp[i, j] += 1e-6
        xm[i, j] -= 1e-6
        fd = (loss(xp) - loss(xm)) / 2e-6
        assert abs(dx.reshape(rows, d)[i, j] - fd) <= 1e-3 * max(1.0, abs(fd))
    # Accumulate adds onto dx.
    dx2 = oracle.layer_norm_backward(r, x, mean, rstd, rows, d, params, np.zeros_like(grads), off, dx=dx, accumulate=True)
    assert np.allclose(dx2, 2 * dx, rtol=1e-6, atol=1e-7)


def test_layer_norm_per_model_parameter_sets():
    # Two models of 30 rows, parameter sets 3 d + 1 floats apart: each row uses its model's set, and
    # each model's gradients land in its own set.
    rows, d, off, k = 60, 16, 2, 2
    params, stride = _ln_params(d, off, models=k, stride=3 * d + 1)
    rng = oracle.Rng(9)
    x, r = rng.gaussian(rows * d), rng.gaussian(rows * d)
    y, mean, rstd = oracle.layer_norm(x, rows, d, params, off, 1e-5, rows_pm=30, stride=stride)
    grads = np.zeros(params.size, np.float32)
    dx = oracle.layer_norm_backward(r, x, mean, rstd, rows, d, params, grads, off, rows_pm=30, stride=stride)
    for m in range(k):
        sl = slice(m * 30 * d, (m + 1) * 30 * d)
        p1 = params[off + m * stride: off + m * stride + 2 * d]
        ym, _, _ = oracle.layer_norm(x[sl], 30, d, p1, 0, 1e-5)
        np.testing.assert_array_equal(y[sl], ym)
        g1 = np.zeros(2 * d, np.float32)
        dxm = oracle.layer_norm_backward(r[sl], x[sl], mean[m * 30:(m + 1) * 30], rstd[m * 30:(m + 1) * 30], 30, d, p1,
                                         g1, 0)
        np.testing.assert_array_equal(dx[sl], dxm)
        np.testing.assert_array_equal(grads[off + m * stride: off + m * stride + 2 * d], g1)


# --------------------------------------------------------------------------- softmax (rows.rs)


def _softmax64(x, t, scale, causal, one):
    rows, n = x.shape
    y = np.zeros((rows, n))
    for r in range(rows):
        lim = (r % t) + 1 if causal else n
        v = scale * x[r, :lim].astype(np.float64)
        if one:
            mx = max(v.max(), 0.0)
            e = np.exp(v - mx)
            y[r, :lim] = e / (e.sum() + np.exp(-mx))
        else:
            e = np.exp(v - v.max())
            y[r, :lim] = e / e.sum()
    return y


@pytest.mark.parametrize("one,amp", [(False, 1.0), (True, 1.0), (True, 40.0), (False, 40.0)])
def test_softmax_forward_and_backward(one, amp):
    t, chunks, scale = 16, 3, 0.125
    rows = chunks * t
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((rows, t)) * amp).astype(np.float32)
    y = oracle.softmax(x, rows, t, t, scale, True, one).reshape(rows, t)
    y64 = _softmax64(x, t, scale, True, one)
    assert np.max(np.abs(y - y64)) < 1e-6
    for r in range(rows):
        assert np.all(y[r, (r % t) + 1:] == 0.0)
        if not one:
            assert abs(y[r].astype(np.float64).sum() - 1.0) < 1e-6
    dy = rng.standard_normal((rows, t)).astype(np.float32)
    dx = oracle.softmax_backward(dy, y, rows, t, scale).reshape(rows, t)
    # Finite differences of L = sum(dy * softmax(scale * x)) in float64.
    eps = 1e-6
    for r, c in [(0, 0), (5, 3), (rows - 1, t - 1), (17, 1)]:
        xp, xm = x.astype(np.float64).copy(), x.astype(np.float64).copy()
        xp[r, c] += eps
        xm[r, c] -= eps
        fd = ((dy * _softmax64(xp, t, scale, True, one)).sum() - (dy * _softmax64(xm, t, scale, True, one)).sum()) / (2 * eps)
        assert abs(dx[r, c] - fd) <= 1e-4 * max(1.0, abs(fd))


@pytest.mark.parametrize("one", [False, True])
def test_attention_fwd_bwd_matches_float64_closed_form(one):
    chunks, t, hd = 3, 32, 16
    scale = 1.0 / math.sqrt(hd)
    rng = np.random.default_rng(4)
    q, k, v, do = (rng.standard_normal((chunks, t, hd)).astype(np.float32) for _ in range(4))
    p, o, dq, dk, dv = oracle.attention_fwd_bwd(q, k, v, do, chunks, t, hd, scale, one)
    Q, K, V, dO = (x.astype(np.float64) for x in (q, k, v, do))
    S = np.einsum("zic,zjc->zij", Q, K) * scale
    S = np.where(np.tril(np.ones((t, t), bool))[None], S, -np.inf)
    mx = S.max(-1, keepdims=True)
    if one:  # softmax1: a phantom logit 0 in every row
        mx = np.maximum(mx, 0.0)
    P = np.exp(S - mx)
    P /= P.sum(-1, keepdims=True) + (np.exp(-mx) if one else 0.0)
    O = P @ V
    dP = dO @ V.transpose(0, 2, 1)
    dV = P.transpose(0, 2, 1) @ dO
    dS = scale * P * (dP - (dP * P).sum(-1, keepdims=True))
    dQ, dK = dS @ K, dS.transpose(0, 2, 1) @ Q
    for got, want in [(p, P), (o, O), (dq, dQ), (dk, dK), (dv, dV)]:
        got = got.reshape(want.shape)
        assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))


# --------------------------------------------------------------------------- 2-bit quantiser (knn.rs:190-225)


def _unpack(codes, d):
    c = np.asarray(codes, np.uint8).reshape(-1, d // 4)
    return np.stack([(c >> (2 * j)) & 3 for j in range(4)], axis=-1).reshape(-1, d).astype(np.int64)


def test_quantizer_hand_computed_rows():
    d = 16
    a = 0.75
    x = np.array([a, -a] * 8, np.float32)
    codes, scales = oracle.quantize_2bit(x, d)
    # sum x^2 / d = a^2, so scale = 0.9957 a; x / scale = +-1.0043 -> u = round(2.504) = 3, round(0.4957) = 0.
    assert scales[0] == np.float32(0.9957) * np.float32(a)
    assert list(_unpack(codes, d)[0]) == [3, 0] * 8
    # packing: code i at byte i/4, bits 2(i%4), low bits first: [3,0,3,0] -> 0b00110011
    assert codes[0, 0] == 0x33
    # zero row: scale floored at 1e-30, every x / scale + 1.5 = 1.5 rounds (away from zero) to 2
    codes, scales = oracle.quantize_2bit(np.zeros(d, np.float32), d)
    assert scales[0] == np.float32(1e-30) and list(_unpack(codes, d)[0]) == [2] * d
    # clamping: one huge component saturates at 3, its negative at 0, small ones sit at 1 or 2
    x = np.array([100.0, -100.0] + [0.01] * 7 + [-0.01] * 7, np.float32)
    u = _unpack(oracle.quantize_2bit(x, d)[0], d)[0]
    assert u[0] == 3 and u[1] == 0 and set(u[2:9]) == {2} and set(u[9:]) == {1}


def test_quantizer_round_half_away_from_zero():
    # Choose a row whose scale is a power of two so that x / scale + 1.5 lands exactly on .5.
    d = 16
    s = np.float32(0.9957) * np.float32(1.0)  # rms 1 -> scale 0.9957
    # components +-1 give rms 1; pick x = +-s so x / scale = +-1 exactly: 2.5 -> 3, 0.5 -> 1 (away from zero)
    x = np.array([s, -s] * 8, np.float32)
    rms = math.sqrt(float((x.astype(np.float32) ** 2).sum()) / d)
    codes, scales = oracle.quantize_2bit(x, d)
    if np.float32(0.9957) * np.float32(rms) == scales[0] and x[0] / scales[0] == 1.0:
        assert list(_unpack(codes, d)[0][:2]) == [3, 1]
    else:  # the chosen row did not produce an exact tie in f32; fall back to the generic property
        u = _unpack(codes, d)[0]
        assert set(u[::2]) <= {2, 3} and set(u[1::2]) <= {0, 1}


def test_quantizer_agrees_with_float64_restatement_away_from_ties():
    d, n = 256, 2000
    keys = np.random.default_rng(5).standard_normal((n, d)).astype(np.float32)
    codes, scales = oracle.quantize_2bit(keys, d)
    k64 = keys.astype(np.float64)
    scale64 = 0.9957 * np.sqrt((k64 ** 2).sum(1) / d)
    assert np.max(np.abs(scales - scale64) / scale64) < 1e-6
    t = k64 / scales[:, None].astype(np.float64) + 1.5
    u64 = np.clip(np.floor(t + 0.5), 0, 3)  # half away from zero for t >= 0 (t < 0 clamps to 0 anyway)
    u = _unpack(codes, d)
    near_tie = np.abs(t - np.round(t - 0.5) - 0.5) < 1e-5
    assert np.all((u == u64) | near_tie)
    assert near_tie.mean() < 1e-3


# --------------------------------------------------------------------------- exact 2-bit scoring contract


def test_query_quantisation_is_exact_power_of_two_scaling():
    rng = np.random.default_rng(2)
    for scale in (1.0, 1e-3, 37.0):
        q = (rng.standard_normal(256) * scale).astype(np.float32)
        Q, prep = oracle.knn_prep_query(q)
        qs = prep.qs
        assert math.frexp(qs)[0] == 0.5  # power of two
        assert 8192 <= np.abs(Q.astype(np.int64)).max() <= 16384 and Q.max() <= 16383
        assert np.all(np.abs(Q.astype(np.float64) * qs - q.astype(np.float64)) <= qs / 2)
        assert prep.sq == int(Q.astype(np.int64).sum())
        assert prep.qn == np.float32(float((Q.astype(np.int64) ** 2).sum())) * np.float32(qs * qs)
    Q, prep = oracle.knn_prep_query(np.zeros(256, np.float32))
    assert prep.qs == 1.0 and not Q.any()


def _brute_force(codes, scales, cell_start, queries, probes, k):
    d = codes.shape[1] * 4
    u = _unpack(codes, d)
    c = 2 * u - 3
    c2 = (c * c).sum(1)
    out_idx, out_dist = [], []
    for qi, q in enumerate(queries):
        Q, prep = oracle.knn_prep_query(q)
        cells = list(dict.fromkeys(int(x) for x in probes[qi]))
        rows = np.concatenate([np.arange(cell_start[cc], cell_start[cc + 1]) for cc in cells]).astype(np.int64)
        dot = c[rows] @ Q.astype(np.int64)  # exact integers
        s = scales[rows]
        t1 = ((s * s) * np.float32(0.25)) * c2[rows].astype(np.float32)
        t3 = (s * np.float32(prep.qs)) * dot.astype(np.float32)
        dist = (t1 - t3).astype(np.float32) + np.float32(0.0)
        order = np.lexsort((rows, dist))[:k]
        idx = np.full(k, -1, np.int64)
        dd = np.full(k, np.inf, np.float32)
        idx[:order.size] = rows[order]
        dd[:order.size] = np.maximum(np.float32(prep.qn) + dist[order], np.float32(0))
        out_idx.append(idx)
        out_dist.append(dd)
    return np.array(out_idx), np.array(out_dist)


def test_knn_search_equals_brute_force_and_handles_edges():
    d, ncells, nq = 256, 12, 9
    rng = np.random.default_rng(8)
    sizes = rng.integers(0, 400, ncells)
    sizes[3] = 5  # a tiny cell
    cell_start = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    keys = rng.standard_normal((cell_start[-1], d)).astype(np.float32)
    codes, scales = oracle.quantize_2bit(keys, d)
    queries = rng.standard_normal((nq, d)).astype(np.float32)
    probes = np.stack([rng.choice(ncells, 4, replace=False) for _ in range(nq)]).astype(np.int32)
    probes[0] = [3, 3, 3, 3]  # fewer than k keys in total: padding; repeated cell scanned once
    probes[1, 2] = probes[1, 0]
    for k in (128, 7):
        idx, dist = oracle.knn_search(codes, scales, cell_start, queries, probes, k)
        widx, wdist = _brute_force(codes, scales, cell_start, queries, probes, k)
        np.testing.assert_array_equal(idx, widx)
        np.testing.assert_array_equal(dist, wdist)
    assert sorted(idx[0][:5]) == list(range(cell_start[3], cell_start[3] + 5))
    idx, dist = oracle.knn_search(codes, scales, cell_start, queries, probes, 128)
    assert np.all(idx[0][5:] == -1) and np.all(np.isinf(dist[0][5:]))


def test_thread_count_does_not_change_results():
    """The all-cores CPU baseline runs the same oracle over several threads: matmul, transpose, gemm and
    knn_search split rows (queries) only, so their outputs are bit-identical to the single-threaded ones."""
    rng = np.random.default_rng(77)
    a = rng.standard_normal((300, 130)).astype(np.float32)
    b = rng.standard_normal((130, 70)).astype(np.float32)
    bias = rng.standard_normal(70).astype(np.float32)
    ref = lambda trans: dict(off=0, stride=0, trans=trans, ld=0, group=1, inner=0)

    def gemm():
        out = np.full(300 * 70 + 70, 0.5, np.float32)
        # Aᵀ read in place from a transposed copy, f16 operands, bias + ReLU, +=, column sums.
        return oracle.gemm(np.ascontiguousarray(a.T), ref(1), b, ref(0), out, ref(0), 1, 300, 130, 70,
                           bias=(bias, 0), relu=True, accumulate=True, col_sum=(300 * 70, 0), f16=True)
    one = oracle.matmul(a, b), oracle.transpose(a), gemm()
    d, ncells, nq = 256, 10, 13
    sizes = rng.integers(50, 300, ncells)
    cell_start = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    codes, scales = oracle.quantize_2bit(rng.standard_normal((cell_start[-1], d)).astype(np.float32), d)
    queries = rng.standard_normal((nq, d)).astype(np.float32)
    probes = np.stack([rng.choice(ncells, 3, replace=False) for _ in range(nq)]).astype(np.int32)
    one_knn = oracle.knn_search(codes, scales, cell_start, queries, probes, 128)
    with oracle.threads(4):
        many = oracle.matmul(a, b), oracle.transpose(a), gemm()
        many_knn = oracle.knn_search(codes, scales, cell_start, queries, probes, 128)
    assert oracle.lib().orc_get_threads() == 1
    for x, y in zip(one + one_knn, many + many_knn):
        np.testing.assert_array_equal(x, y)


def test_knn_masked_search_equals_brute_force_over_the_allowed_keys():
    d, n, nq = 256, 3000, 12
    rng = np.random.default_rng(41)
    keys = rng.standard_normal((n, d)).astype(np.float32)
    codes, scales = oracle.quantize_2bit(keys, d)
    queries = rng.standard_normal((nq, d)).astype(np.float32)
    lo = rng.integers(0, n, nq)
    hi = np.minimum(lo + rng.integers(0, 900, nq), n + 50)  # some ranges run past the store (clipped)
    lo[0], hi[0] = 100, 100        # empty range: only the always-visible prefix
    lo[1], hi[1] = 2990, 5000      # 10 keys
    for always, k in ((0, 128), (37, 128), (500, 7)):
        idx, dist = oracle.knn_search_masked(codes, scales, queries, lo, hi, always, k)
        # The brute force over the same allowed keys, written as one "cell" per query.
        for qi in range(nq):
            allowed = [g for g in range(n) if g < always or lo[qi] <= g < hi[qi]]
            cs = np.array([0, len(allowed)], np.int64)
            sel = np.array(allowed, np.int64)
            widx, wdist = _brute_force(codes[sel], scales[sel], cs, queries[qi:qi + 1], np.zeros((1, 1), np.int32), k)
            got = np.where(widx[0] >= 0, sel[np.maximum(widx[0], 0)], -1) if sel.size else widx[0]
            np.testing.assert_array_equal(idx[qi], got)
            np.testing.assert_array_equal(dist[qi], wdist[0])
    idx, _ = oracle.knn_search_masked(codes, scales, queries, lo, hi, 0, 128)
    assert np.all(idx[0] == -1)
    assert sorted(idx[1][:10]) == list(range(2990, 3000)) and np.all(idx[1][10:] == -1)
    # A range that is exactly one cell gives the IVF search's answer for that cell.
    cs = np.array([0, 700, 1900, 3000], np.int64)
    idx, dist = oracle.knn_search_masked(codes, scales, queries[:3], [700] * 3, [1900] * 3, 0, 128)
    widx, wdist = oracle.knn_search(codes, scales, cs, queries[:3], np.ones((3, 1), np.int32), 128)
    np.testing.assert_array_equal(idx, widx)
    np.testing.assert_array_equal(dist, wdist)


def test_query_quantisation_of_subnormal_queries():
    rng = np.random.default_rng(42)
    for scale in (2.0 ** -120, 2.0 ** -135, 2.0 ** -148):
        q = (rng.standard_normal(256) * scale).astype(np.float32)
        Q, prep = oracle.knn_prep_query(q)
        mx = float(np.max(np.abs(q)))
        e = math.frexp(mx)[1]
        assert prep.qe == e - 14
        err = np.abs(np.ldexp(Q.astype(np.float64), prep.qe) - q.astype(np.float64))
        assert np.all(err <= np.ldexp(0.5, prep.qe))
        assert np.max(np.abs(Q)) >= 8192


def test_knn_integer_dot_is_exact_and_close_to_the_references_f16_scoring():
    d = 256
    rng = np.random.default_rng(11)
    keys = rng.standard_normal((300, d)).astype(np.float32)
    codes, scales, norms = oracle.quantize_2bit(keys, d, with_norm=True)
    q = rng.standard_normal(d).astype(np.float32)
    Q, prep = oracle.knn_prep_query(q)
    dists = oracle.knn_dists(codes, scales, d, 0, 300, q)
    u = _unpack(codes, d)
    khat = (u - 1.5) * scales[:, None].astype(np.float64)
    qhat = Q.astype(np.float64) * prep.qs
    exact = (khat ** 2).sum(1) - 2 * khat @ qhat
    assert np.max(np.abs(dists - exact) / (1 + np.abs(exact))) < 1e-6
    # The reference scores f16(q) against f16((u - 1.5) s) with its stored norm; the
    # contract stays within the 2e-3 * (1 + d) its own IVF test allows (ivf.rs:770).
    for r in range(300):
        ref = oracle.knn_ref_f16_dist(codes[r], scales[r], norms[r], q)
        ours = float(prep.qn) + float(dists[r])
        assert abs(ours - ref) < 2e-3 * (1 + abs(ref))


# --------------------------------------------------------------------------- probe selection


def _dequantised(x):
    """x [n, d] f32 -> each row as the scan's quantiser represents it, in float64 (exact)."""
    out = np.empty(x.shape, np.float64)
    for i, row in enumerate(x):
        Q, prep = oracle.knn_prep_query(row)
        out[i] = Q.astype(np.float64) * float(prep.qs)
    return out


def _rank(d2, nprobe):
    """The nprobe smallest of each row of d2 by (value, column), as int32."""
    cols = np.arange(d2.shape[1])
    return np.stack([np.lexsort((cols, row))[:nprobe] for row in d2]).astype(np.int32)


def test_centroid_prep_is_the_query_quantiser_with_exact_norms():
    rng = np.random.default_rng(21)
    cent = rng.standard_normal((40, 256)).astype(np.float32)
    cent[3] = 0.0
    cent[7] *= np.float32(2.0 ** -30)
    cent[9] *= np.float32(2.0 ** 30)
    C, cexp, cnorm = oracle.knn_centroid_prep(cent)
    for c in range(40):
        Q, prep = oracle.knn_prep_query(cent[c])
        np.testing.assert_array_equal(C[c], Q)
        assert 2.0 ** int(cexp[c]) == float(prep.qs)
    deq = C.astype(np.float64) * np.exp2(cexp.astype(np.float64))[:, None]
    np.testing.assert_array_equal(cnorm, (deq ** 2).sum(1))  # every term and partial sum is exact
    assert cnorm[3] == 0.0 and cexp[3] == 0
    rel = np.abs(cnorm - (cent.astype(np.float64) ** 2).sum(1)) / np.maximum((cent.astype(np.float64) ** 2).sum(1), 1e-300)
    assert np.all(rel[np.arange(40) != 3] < 2.0 ** -11)


@pytest.mark.parametrize("scale_spread", [False, True])
def test_probe_ranks_by_the_dequantised_distance(scale_spread):
    rng = np.random.default_rng(22)
    nlist, nq, d, nprobe = 300, 24, 256, 16
    cent = rng.standard_normal((nlist, d)).astype(np.float32)
    if scale_spread:  # centroid and query magnitudes from 2^-40 to 2^40
        cent *= np.exp2(rng.integers(-40, 41, nlist)).astype(np.float32)[:, None]
    queries = rng.standard_normal((nq, d)).astype(np.float32)
    if scale_spread:
        queries *= np.exp2(rng.integers(-40, 41, nq)).astype(np.float32)[:, None]
    probes = oracle.knn_probe(cent, queries, nprobe)
    qh, ch = _dequantised(queries), _dequantised(cent)
    d2 = ((qh[:, None, :] - ch[None, :, :]) ** 2).sum(2)  # |q^ - c^|^2, a different expression of the same order
    want = _rank(d2, nprobe)
    # Rows whose float64 sums leave a near-tie ambiguous are rare; none at this seed.
    np.testing.assert_array_equal(probes, want)


def test_probe_agrees_with_unquantised_distance_where_the_gap_is_clear():
    rng = np.random.default_rng(23)
    nlist, nq, d, nprobe = 500, 40, 256, 8
    cent = rng.standard_normal((nlist, d)).astype(np.float32)
    queries = (cent[rng.integers(0, nlist, nq)] + 0.7 * rng.standard_normal((nq, d))).astype(np.float32)
    probes = oracle.knn_probe(cent, queries, nprobe)
    true = ((queries.astype(np.float64)[:, None, :] - cent.astype(np.float64)[None]) ** 2).sum(2)
    checked = 0
    for i in range(nq):
        srt = np.sort(true[i])
        if srt[nprobe] - srt[nprobe - 1] > 1e-2:  # the quantisation moves d2 by < 1e-2 here
            assert set(probes[i]) == set(np.argsort(true[i])[:nprobe])
            checked += 1
    assert checked > nq // 2


def test_probe_query_equal_to_a_centroid_and_duplicate_centroids():
    rng = np.random.default_rng(24)
    cent = rng.standard_normal((64, 256)).astype(np.float32)
    cent[40] = cent[5]
    cent[50] = cent[5]
    queries = np.stack([cent[17], cent[5], cent[5] + 1e-3 * rng.standard_normal(256).astype(np.float32)])
    p = oracle.knn_probe(cent, queries, 4)
    assert p[0, 0] == 17
    assert list(p[1, :3]) == [5, 40, 50]  # equal dd: the lower id first
    assert list(p[2, :3]) == [5, 40, 50]
    assert list(oracle.knn_probe(cent, queries, 2)[1]) == [5, 40]


def test_probe_is_covariant_under_centroid_permutation_and_full_sort_at_nprobe_nlist():
    rng = np.random.default_rng(25)
    nlist = 16
    cent = rng.standard_normal((nlist, 256)).astype(np.float32)
    queries = rng.standard_normal((10, 256)).astype(np.float32)
    perm = rng.permutation(nlist)
    p = oracle.knn_probe(cent, queries, 5)
    pp = oracle.knn_probe(cent[perm], queries, 5)
    np.testing.assert_array_equal(perm[pp], p)
    full = oracle.knn_probe(cent, queries, nlist)
    for row in full:
        assert sorted(row) == list(range(nlist))
    # A zero query ranks the cells by centroid norm (then id).
    _, _, cnorm = oracle.knn_centroid_prep(cent)
    z = oracle.knn_probe(cent, np.zeros((1, 256), np.float32), nlist)
    np.testing.assert_array_equal(z[0], np.lexsort((np.arange(nlist), cnorm)))


def test_quantizer_norm_is_the_f16_dequantised_norm_summed_in_order():
    # knn.rs:216: sum over dims, in order, of f16((u - 1.5) * scale)^2 in f32.
    rng = np.random.default_rng(43)
    keys = rng.standard_normal((50, 256)).astype(np.float32)
    keys[0] *= np.float32(1e-3)
    keys[1] *= np.float32(300.0)
    codes, scales, norms = oracle.quantize_2bit(keys, 256, with_norm=True)
    u = _unpack(codes, 256)
    deq = ((u.astype(np.float32) - np.float32(1.5)) * scales[:, None]).astype(np.float16).astype(np.float32)
    want = np.cumsum(deq * deq, axis=1, dtype=np.float32)[:, -1]
    np.testing.assert_array_equal(norms, want)
