"""GEMM parity through the C ABI against the CPU oracle (gpu_step::matmul semantics).

Tolerances (scale-relative: max|gpu - cpu| / max|cpu|, as matmul.rs:1077-1086):
  f32 route         <= 1e-5 vs the oracle
  f16-in route      <= 1e-5 vs the oracle on f16-rounded operands (same products,
                       different summation order) and <= 2e-3 vs the f32 oracle
  column sums       <= 1e-4 (f32) / 1e-3 (f16) of their scale, as matmul.rs:1081
"""
import random

import numpy as np
import pytest
import torch

import oracle
import scratchtape_amd as st
from scratchtape_amd import Epilogue, MatRef
from scratchtape_amd.tensor import ndarray_matmul

pytestmark = pytest.mark.gpu

# (batch, m, k, n, trans_a, trans_b, bias, relu, mask, residual, accumulate): matmul.rs:966-1007
CASES_F16 = [
    (1, 128, 64, 64, False, False, False, False, False, False, False),
    (1, 128, 64, 64, True, False, False, False, False, False, False),
    (1, 128, 64, 64, False, True, False, False, False, False, False),
    (1, 128, 64, 64, True, True, False, False, False, False, False),
    (3, 64, 96, 128, False, True, True, True, False, False, False),
    (3, 64, 64, 64, True, False, False, False, False, True, True),
    (2, 128, 32, 128, False, False, True, False, True, True, True),
    (1, 128, 64, 64, False, False, False, False, True, False, False),
    (1, 256, 128, 256, False, True, False, False, False, False, False),
    (1, 256, 128, 128, False, False, True, True, False, False, False),
    (2, 128, 64, 96, False, False, True, True, False, True, False),
    (3, 64, 64, 64, True, False, False, False, False, False, True),
    (2, 128, 64, 96, False, True, False, False, False, False, True),
    (1, 128, 1024, 128, True, False, False, False, False, False, False),
    (1, 128, 1024, 128, True, False, False, False, False, False, True),
    (3, 64, 1024, 64, True, False, False, False, False, False, True),
    (1, 64, 256, 64, True, False, False, False, False, False, False),
    (1, 64, 256, 64, False, False, False, False, False, False, True),
    (1, 70, 64, 64, False, False, True, False, False, False, False),
    (1, 64, 48, 64, False, False, True, False, False, False, False),
    (2, 33, 17, 65, True, False, True, True, True, True, True),
]
CASES_F32 = [
    (1, 70, 35, 20, False, False, False, False, False, False, False),
    (1, 70, 35, 20, True, False, False, False, False, False, False),
    (1, 70, 35, 20, False, True, False, False, False, False, False),
    (1, 70, 35, 20, True, True, False, False, False, False, False),
    (3, 33, 17, 65, False, True, True, True, False, False, False),
    (3, 64, 64, 64, True, False, False, False, False, True, True),
    (1, 512, 128, 384, False, False, True, False, False, False, False),
    (1, 128, 512, 384, True, False, False, False, False, False, True),
    (1, 128, 512, 128, True, False, False, False, False, False, True),
    (1, 70, 300, 20, True, False, False, False, False, False, False),
    (3, 128, 512, 128, True, False, False, False, False, False, True),
    (2, 70, 300, 20, True, False, False, False, False, False, False),
    (1, 512, 256, 128, False, True, False, False, False, False, False),
    (64, 64, 16, 64, False, True, False, False, False, False, False),
    (64, 64, 64, 16, False, False, False, False, False, False, False),
    (1, 512, 128, 256, False, False, True, True, False, False, False),
    (1, 512, 256, 128, False, False, True, False, False, True, False),
    (1, 512, 128, 256, False, True, False, False, True, False, False),
    (2, 33, 17, 65, True, False, True, True, True, True, True),
]


def rel_err(got, want):
    scale = float(np.max(np.abs(want))) if want.size else 0.0
    return float(np.max(np.abs(got - want))) / max(scale, 1e-30)


def prep_case(dev, ci, case, use_f16, aligned16=False, packed=False):
    """Buffers, the matmul_with arguments and the oracle's answers for one case.
    aligned16: every operand, stride and epilogue tensor on 16-byte boundaries (the layouts the
    LDS-DMA kernels take); packed: out matrices back to back (the layout split-k needs)."""
    batch, m, k, n, ta, tb, has_bias, relu, has_mask, has_res, acc = case
    rng = oracle.Rng(5 + ci)
    gauss = rng.gaussian
    aligned = use_f16 and ci % 2 == 1
    a_off, b_off, o_off, bias_off, m_off, r_off = 3, 5, (8 if aligned else 7), 2, 6, 1
    sa, sb, so = m * k + 1, (k * n + 2 if batch > 1 else 0), m * n + (0 if aligned else 3)
    if aligned16:
        a_off, b_off, o_off, bias_off, m_off, r_off = 4, 8, 12, 2, 16, 20
        sa, sb, so = m * k + 4, (k * n + 8 if batch > 1 else 0), m * n + (0 if packed else 4)
    a = gauss(a_off + batch * sa)
    b = gauss(b_off + max(batch, 1) * max(sb, k * n))
    bias_stride = n + 1 if batch > 1 else 0
    bias = gauss(bias_off + batch * (n + 1))
    res = gauss(r_off + batch * so)
    mask = gauss(m_off + batch * so)
    cs_off, cs_stride = o_off + batch * so + 5, n + 3
    out0 = gauss(cs_off + batch * cs_stride + 2)

    f16 = use_f16 and st.f16_route(m, k, n, col_sum=True, b_trans=tb)
    kw = dict(bias=(bias, bias_off) if has_bias else None, bias_stride=bias_stride, relu=relu,
              mask=(mask, m_off) if has_mask else None, residual=(res, r_off) if has_res else None,
              accumulate=acc, col_sum=(cs_off, cs_stride))
    refs = dict(a=dict(off=a_off, stride=sa, trans=ta), b=dict(off=b_off, stride=sb, trans=tb),
                out=dict(off=o_off, stride=so))
    want32 = oracle.gemm(a, refs["a"], b, refs["b"], out0.copy(), refs["out"], batch, m, k, n, **kw)
    want16 = oracle.gemm(a, refs["a"], b, refs["b"], out0.copy(), refs["out"], batch, m, k, n, f16=True, **kw)

    T = lambda x: torch.from_numpy(x).to(dev)
    ah, bh, biash, maskh, resh, oh = T(a), T(b), T(bias), T(mask), T(res), T(out0)
    epi = Epilogue(bias=(biash, bias_off) if has_bias else None, bias_stride=bias_stride, relu=relu,
                   mask=(maskh, m_off) if has_mask else None, residual=(resh, r_off) if has_res else None,
                   accumulate=acc, col_sum=(cs_off, cs_stride))
    call = (MatRef(ah, off=a_off, stride=sa, trans=ta), MatRef(bh, off=b_off, stride=sb, trans=tb),
            MatRef(oh, off=o_off, stride=so), batch, m, k, n, epi, use_f16)
    return dict(call=call, oh=oh, out0=out0, want16=want16, want32=want32, cs_off=cs_off, f16=f16,
                what=f"case {ci} {case} f16_route={f16}")


def check_case(p, got=None):
    got = p["oh"].cpu().numpy() if got is None else got
    body, cs = slice(0, p["cs_off"]), slice(p["cs_off"], None)
    what = p["what"]
    if p["f16"]:
        assert rel_err(got[body], p["want16"][body]) <= 1e-5, what
        assert rel_err(got[body], p["want32"][body]) <= 2e-3, what
        assert rel_err(got[cs], p["want32"][cs]) <= 1e-3, what
    else:
        assert rel_err(got[body], p["want32"][body]) <= 1e-5, what
        assert rel_err(got[cs], p["want32"][cs]) <= 1e-4, what


def run_case(dev, ci, case, use_f16, aligned16=False, packed=False):
    p = prep_case(dev, ci, case, use_f16, aligned16, packed)
    st.matmul_with(*p["call"])
    check_case(p)


# Shapes for the LDS-DMA kernel (m, n tile-divisible, k % 32 == 0), run with 16-byte aligned
# layouts: every epilogue term, batched strides, and split-k (few tiles, free epilogue) with
# accumulate and column sums, batched and with many slices.
# (batch, m, k, n, bias, relu, mask, residual, accumulate, packed)
DMA_CASES = [
    (2, 128, 96, 128, True, True, False, False, False, False),
    (2, 128, 64, 64, True, False, True, True, True, False),
    (1, 256, 128, 192, False, True, True, False, True, False),
    (1, 256, 2048, 128, False, False, False, False, True, True),
    (3, 64, 1024, 64, False, False, False, False, True, True),
    (1, 64, 4096, 64, False, False, False, False, False, True),
    # 32 slices of 256 (long-k split rule): the split sum's loads go out in two blocks of 16
    (1, 64, 8192, 64, False, False, False, False, True, True),
    # m, n multiples of 32 but not of 64: the f32 route's 32 x 32 tiles (the f16 route takes k_gemm)
    (1, 96, 256, 160, True, True, True, True, True, False),
    (2, 32, 1024, 96, False, False, False, False, True, True),
    # n = 48: no DMA tile fits; batched 16 x 16 tiles (k_gemm_tiny), f32 and f16 routes
    (2, 64, 256, 48, True, False, True, False, True, False),
]


@pytest.mark.parametrize("use_f16", [False, True])
@pytest.mark.parametrize("tt", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("ci", range(len(DMA_CASES)))
def test_matmul_aligned_layouts_match_oracle(dev, ci, tt, use_f16):
    batch, m, k, n, bias, relu, mask, res, acc, packed = DMA_CASES[ci]
    case = (batch, m, k, n, tt[0], tt[1], bias, relu, mask, res, acc)
    run_case(dev, 100 + ci, case, use_f16, aligned16=True, packed=packed)


@pytest.mark.parametrize("ci", range(len(CASES_F32)))
def test_matmul_f32_matches_oracle(dev, ci):
    run_case(dev, ci, CASES_F32[ci], False)


@pytest.mark.parametrize("ci", range(len(CASES_F16)))
def test_matmul_f16_matches_oracle(dev, ci):
    run_case(dev, ci, CASES_F16[ci], True)


def check_head_views(dev, bsz, heads, t, w, use_f16, tol):
    """matmul.rs:1113-1195: scores = Q Kᵀ from a fused QKV buffer, ctx += P V into merged heads,
    dV += Pᵀ dCtx into V's columns of the fused buffer."""
    hw, fused = heads * w, 3 * heads * w
    batch = bsz * heads
    rng = oracle.Rng(9)
    qkv, p, ctx0, dctx = (rng.gaussian(n) for n in (bsz * t * fused, batch * t * t, bsz * t * hw, bsz * t * hw))
    T = lambda x: torch.from_numpy(x).to(dev)
    hv = lambda col0, cols: dict(off=col0, stride=t * cols, ld=cols, group=heads, inner=w)

    want = np.zeros(batch * t * t, np.float32)
    oracle.gemm(qkv, hv(0, fused), qkv, dict(hv(hw, fused), trans=True), want, dict(stride=t * t), batch, t, w, t,
                f16=use_f16)
    sh = torch.zeros(batch * t * t, device=dev)
    st.matmul_with(MatRef.heads(T(qkv), 0, fused, t, heads, w),
                   MatRef.heads(T(qkv), hw, fused, t, heads, w).with_(trans=True),
                   MatRef(sh, stride=t * t), batch, t, w, t, None, use_f16)
    assert rel_err(sh.cpu().numpy(), want) <= tol, "scores"

    want = ctx0.copy()
    oracle.gemm(p, dict(stride=t * t), qkv, hv(2 * hw, fused), want, hv(0, hw), batch, t, t, w, accumulate=True,
                f16=use_f16)
    ch = T(ctx0)
    st.matmul_with(MatRef(T(p), stride=t * t), MatRef.heads(T(qkv), 2 * hw, fused, t, heads, w),
                   MatRef.heads(ch, 0, hw, t, heads, w), batch, t, t, w, Epilogue(accumulate=True), use_f16)
    assert rel_err(ch.cpu().numpy(), want) <= tol, "ctx"

    want = qkv.copy()
    oracle.gemm(p, dict(stride=t * t, trans=True), dctx, hv(0, hw), want, hv(2 * hw, fused), batch, t, t, w,
                accumulate=True, f16=use_f16)
    gh = T(qkv)
    st.matmul_with(MatRef(T(p), stride=t * t, trans=True), MatRef.heads(T(dctx), 0, hw, t, heads, w),
                   MatRef.heads(gh, 2 * hw, fused, t, heads, w), batch, t, t, w, Epilogue(accumulate=True), use_f16)
    assert rel_err(gh.cpu().numpy(), want) <= tol, "dV"


def test_head_views_f32(dev):
    check_head_views(dev, 2, 3, 5, 4, False, 1e-5)


def test_head_views_f16_attention_shapes(dev):
    # head width 64, t 128 (the attention configuration), where every one of the three takes the f16 route
    assert st.f16_route(128, 64, 128) and st.f16_route(128, 128, 64)
    check_head_views(dev, 2, 4, 128, 64, True, 1e-5)


def test_ndarray_matmul_known_answer_and_random():
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    np.testing.assert_array_equal(ndarray_matmul(a, b), [[58, 64], [139, 154]])
    # gpu.rs:186-199: 37x53x29 from Rng(42), next_f32()*2-1
    rng = oracle.Rng(42)
    a = rng.uniform(37 * 53).reshape(37, 53)
    b = rng.uniform(53 * 29).reshape(53, 29)
    assert rel_err(ndarray_matmul(a, b), oracle.matmul(a, b)) <= 1e-5


def test_integer_inputs_are_exact_on_both_routes(dev):
    # Integer-valued operands: every partial sum is an exact f32 integer, so the
    # GPU must equal the CPU bit for bit whatever its summation order.
    rng = np.random.default_rng(0)
    m, k, n = 256, 512, 192
    a = rng.integers(-8, 9, (m, k)).astype(np.float32)
    b = rng.integers(-8, 9, (k, n)).astype(np.float32)
    want = oracle.matmul(a, b)
    for use_f16 in (False, True):
        out = torch.zeros(m * n, device=dev)
        st.matmul_with(MatRef(torch.from_numpy(a).to(dev)), MatRef(torch.from_numpy(b).to(dev)), MatRef(out),
                       1, m, k, n, None, use_f16)
        np.testing.assert_array_equal(out.cpu().numpy().reshape(m, n), want)


def tape_forms(dev, m, k, n, use_f16, seed):
    """C = A·B, dA = dC·Bᵀ, dB = Aᵀ·dC (tape.rs:504-510) with A [m,k], B [k,n], dC [m,n] uniform [-1,1]."""
    rng = oracle.Rng(seed)
    A, B, dC = rng.uniform(m * k).reshape(m, k), rng.uniform(k * n).reshape(k, n), rng.uniform(m * n).reshape(m, n)
    T = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    Ah, Bh, dCh = T(A), T(B), T(dC)
    C, dA, dB = (torch.zeros(s, device=dev) for s in (m * n, m * k, k * n))
    st.matmul_with(MatRef(Ah), MatRef(Bh), MatRef(C), 1, m, k, n, None, use_f16)
    st.matmul_with(MatRef(dCh), MatRef(Bh, trans=True), MatRef(dA), 1, m, n, k, None, use_f16)
    st.matmul_with(MatRef(Ah, trans=True), MatRef(dCh), MatRef(dB), 1, k, m, n, None, use_f16)
    r = oracle.round_f16 if use_f16 else (lambda x: x)
    wants = [oracle.matmul(r(A), r(B)), oracle.matmul(r(dC), oracle.transpose(r(B))),
             oracle.matmul(oracle.transpose(r(A)), r(dC))]
    wants32 = [oracle.matmul(A, B), oracle.matmul(dC, oracle.transpose(B)), oracle.matmul(oracle.transpose(A), dC)]
    for name, got, want, want32 in zip(["C", "dA", "dB"], [C, dA, dB], wants, wants32):
        g = got.cpu().numpy().reshape(want.shape)
        assert rel_err(g, want) <= 1e-5, (name, m, k, n, use_f16)
        if use_f16:
            assert rel_err(g, want32) <= 2e-3, (name, m, k, n)


@pytest.mark.parametrize("use_f16", [False, True])
def test_tape_forms_256_cube(dev, use_f16):
    tape_forms(dev, 256, 256, 256, use_f16, 42)


@pytest.mark.parametrize("use_f16", [False, True])
def test_tape_backward_rectangular(dev, use_f16):
    # dA[4096,256] = dC[4096,1024]·Bᵀ and dB[256,1024] = Aᵀ[256,4096]·dC
    tape_forms(dev, 4096, 256, 1024, use_f16, 43)


STEP_SHAPES = [(4096, 256, 768), (4096, 256, 256), (4096, 256, 1024), (4096, 1024, 256)]


@pytest.mark.parametrize("shape", STEP_SHAPES)
@pytest.mark.parametrize("use_f16", [False, True])
def test_step_set_shapes(dev, shape, use_f16):
    m, k, n = shape
    tape_forms(dev, m, k, n, use_f16, 100 + k + n)


def test_bad_arguments_raise_with_the_reference_message(dev):
    x = torch.zeros(16, device=dev)
    with pytest.raises(st.ScratchtapeError, match="out is stored row-major"):
        st.matmul(MatRef(x), MatRef(x), MatRef(x, trans=True), 1, 4, 4, 4)


# Grouped launches (st_matmul_grouped): GEMMs that tile by 128 x 128 share one
# persistent launch per route; the others (last two) run one by one.
# (batch, m, k, n, trans_a, trans_b, bias, relu, mask, residual, accumulate, packed)
GROUP_CASES = [
    (1, 256, 256, 384, False, False, True, True, False, False, False, False),
    (1, 128, 1024, 256, True, False, False, False, False, False, True, True),
    (2, 128, 128, 128, False, True, False, False, True, True, False, False),
    (1, 384, 512, 128, True, True, True, False, False, False, False, False),
    (3, 128, 256, 128, True, False, False, False, False, False, True, True),
    (1, 128, 128, 256, False, False, False, False, False, False, True, False),
    (1, 256, 4096, 128, True, False, False, False, False, False, False, True),
    (1, 64, 64, 64, False, False, True, False, False, False, False, False),
    (1, 70, 35, 20, True, False, False, False, False, True, False, False),
]


def group_preps(dev, use_f16, idx):
    out = []
    for i in idx:
        c = GROUP_CASES[i]
        out.append(prep_case(dev, 200 + i, c[:11], use_f16, aligned16=True, packed=c[11]))
    return out


@pytest.mark.parametrize("use_f16", [False, True])
def test_grouped_matches_oracle(dev, use_f16):
    ps = group_preps(dev, use_f16, range(len(GROUP_CASES)))
    st.matmul_grouped([p["call"] for p in ps])
    for p in ps:
        check_case(p)


@pytest.mark.parametrize("use_f16", [False, True])
def test_grouped_with_256_row_tiles_matches_oracle(dev, use_f16):
    # A 4096 x 2048 GEMM gives the route 256 tiles of 256 rows, so every GEMM of the
    # group whose m is a multiple of 256 (cases 0 and 6) runs on the 8-wave 256-row
    # kernel, the others on the 128-row one.
    ps = group_preps(dev, use_f16, range(len(GROUP_CASES)))
    ps.append(prep_case(dev, 300, (1, 4096, 128, 2048, False, False, True, False, False, False, True), use_f16,
                        aligned16=True))
    st.matmul_grouped([p["call"] for p in ps])
    for p in ps:
        check_case(p)


@pytest.mark.parametrize("use_f16", [False, True])
def test_grouped_of_one_and_repeated(dev, use_f16):
    # A group of one (split-k over many slices: the only GEMM of the launch), then
    # the same group again: the second call starts from the first call's output.
    ps = group_preps(dev, use_f16, [6])
    st.matmul_grouped([ps[0]["call"]])
    check_case(ps[0])
    ps = group_preps(dev, use_f16, [1, 4])
    for _ in range(2):
        st.matmul_grouped([p["call"] for p in ps])
    for p in ps:
        # accumulate: out = out0 + 2 * product (and column sums twice); the route's
        # product is the f16-rounded one on the f16 route, column sums are f32
        prod = p["want32"] - p["out0"]
        if p["f16"]:
            body = slice(0, p["cs_off"])
            prod[body] = p["want16"][body] - p["out0"][body]
        check_case(p, got=p["oh"].cpu().numpy() - prod)


@pytest.mark.parametrize("use_f16", [False, True])
def test_grouped_equals_single_calls_bit_for_bit_without_split(dev, use_f16):
    # GEMMs with a bias, mask or residual never split: each output element is
    # the same sequence of operations in the grouped and the single-GEMM kernel.
    idx = [0, 2, 3]
    ps = group_preps(dev, use_f16, idx)
    st.matmul_grouped([p["call"] for p in ps])
    got = [p["oh"].cpu().numpy() for p in ps]
    for p, g in zip(ps, got):
        p["oh"].copy_(torch.from_numpy(p["out0"]).to(dev))
        st.matmul_with(*p["call"])
        np.testing.assert_array_equal(g, p["oh"].cpu().numpy(), err_msg=p["what"])


def random_case(rnd):
    """A GEMM case (and whether its outputs are packed) drawn by rnd: tile-divisible or ragged
    shapes, batches, transposes, every epilogue term; at most 2^24 multiply-adds."""
    if rnd.random() < 0.2:
        m, k, n = rnd.randint(1, 160), rnd.randint(1, 300), rnd.randint(1, 160)
    else:
        m, n = rnd.choice([64, 128, 256, 384]), rnd.choice([64, 128, 256])
        k = rnd.choice([32, 96, 256, 512, 1024, 2048])
    batch = rnd.choice([1, 1, 2, 3])
    while batch * m * n * k > (1 << 24) and k > 32:
        k //= 2
    epi = [rnd.random() < 0.3 for _ in range(5)]  # bias, relu, mask, residual, accumulate
    case = (batch, m, k, n, rnd.random() < 0.5, rnd.random() < 0.5, *epi)
    return case, not any(epi[:4]) and rnd.random() < 0.7


def test_random_single_calls_match_oracle(dev):
    # Seeded random cases one call each: the dispatch's tile, split-k and small-product choices.
    rnd = random.Random(12)
    for ci in range(24):
        case, packed = random_case(rnd)
        p = prep_case(dev, 700 + ci, case, ci % 2 == 1, aligned16=True, packed=packed)
        st.matmul_with(*p["call"])
        check_case(p)


def test_grouped_random_groups_match_oracle(dev):
    # Seeded random groups of 1-5 GEMMs on both routes, outputs packed (split-k allowed) or not.
    rnd = random.Random(11)
    for gi in range(12):
        ps = []
        for i in range(rnd.randint(1, 5)):
            case, packed = random_case(rnd)
            ps.append(prep_case(dev, 500 + 8 * gi + i, case, gi % 2 == 1, aligned16=True, packed=packed))
        st.matmul_grouped([p["call"] for p in ps])
        for p in ps:
            check_case(p)


@pytest.mark.parametrize("use_f16", [False, True])
def test_grouped_step_set_matches_the_oracle(dev, use_f16):
    """The 15 GEMMs of a d_model-256 step (T = 4096) as one group -- the call the benchmark times -- against the
    oracle's NdArray::matmul restatement (with the tape's explicit transposes), every GEMM: f16 route 1e-5 on
    f16-rounded operands and 2e-3 on the f32 ones, f32 route 1e-5 (scale-relative, matmul.rs:1077-1086)."""
    T, calls, checks = 4096, [], []
    g = torch.Generator(device="cpu").manual_seed(3)
    for K, N in [(256, 768), (256, 256), (256, 1024), (1024, 256), (256, 256)]:
        X, W, dY = (torch.randn(s, generator=g) for s in ((T, K), (K, N), (T, N)))
        W *= 0.02
        Xd, Wd, dYd = X.to(dev), W.to(dev), dY.to(dev)
        Y, dX, dW = torch.zeros(T, N, device=dev), torch.zeros(T, K, device=dev), torch.zeros(K, N, device=dev)
        calls += [(MatRef(Xd), MatRef(Wd), MatRef(Y), 1, T, K, N, None, use_f16),
                  (MatRef(dYd), MatRef(Wd, trans=True), MatRef(dX), 1, T, N, K, None, use_f16),
                  (MatRef(Xd, trans=True), MatRef(dYd), MatRef(dW), 1, K, T, N, None, use_f16)]
        x, w, dy = X.numpy(), W.numpy(), dY.numpy()
        checks += [(Y, x, w), (dX, dy, oracle.transpose(w)), (dW, oracle.transpose(x), dy)]
    st.matmul_grouped(calls)
    torch.cuda.synchronize()
    with oracle.threads(8):
        for i, (out, a, b) in enumerate(checks):
            got = out.cpu().numpy()
            want = oracle.matmul(a, b)
            err = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
            assert err <= (2e-3 if use_f16 else 1e-5), (i, err)
            if use_f16:
                want16 = oracle.matmul(oracle.round_f16(a), oracle.round_f16(b))
                err16 = float(np.max(np.abs(got - want16)) / np.max(np.abs(want16)))
                assert err16 <= 1e-5, (i, err16)


def test_grouped_step_set_with_tape_epilogues(dev):
    """The C3 set at T = 4096 as one grouped call with the device tape's epilogues (gpu_step/tape.rs:180-189,
    324-347): forward + bias (+ ReLU on FFN1, + residual after attention and FFN), dW += with the bias gradient as
    column sums; every product within 1e-5 of the oracle on f16-rounded operands, the column sums within 1e-4."""
    import bench
    ss = bench.StepSet(dev, epilogues=True)
    err, cs_err = bench.check_epilogue_set(ss)
    assert err <= 1e-5, err
    assert cs_err <= 1e-4, cs_err
