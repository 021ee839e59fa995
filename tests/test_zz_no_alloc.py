"""st_matmul_grouped_noalloc (no reference counterpart: st_matmul_grouped for callers that cannot allocate) against
st_matmul_grouped, through the C ABI: the same kernels and split points, so the outputs must agree bit for bit.  Two
calls in a row, the second on a smaller step set, each checked against the allocating entry point on fresh
outputs; and a group whose split-k partials exceed the fixed scratch is refused before anything runs."""
import numpy as np
import pytest
import torch

import scratchtape_amd as st
from scratchtape_amd import Epilogue, MatRef

pytestmark = pytest.mark.gpu


def step_set(dev, T, use_f16, seed):
    """The 15 GEMMs of a d_model-256 step with T tokens (the dW GEMMs, k = T, split over k)."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    calls, outs = [], []
    for K, N in [(256, 768), (256, 256), (256, 1024), (1024, 256), (256, 256)]:
        X, W, dY = (torch.randn(s, generator=gen).to(dev) for s in ((T, K), (K, N), (T, N)))
        Y, dX, dW = (torch.full(s, 7.0, device=dev) for s in ((T, N), (T, K), (K, N)))
        calls += [(MatRef(X), MatRef(W), MatRef(Y), 1, T, K, N, None, use_f16),
                  (MatRef(dY), MatRef(W, trans=True), MatRef(dX), 1, T, N, K, None, use_f16),
                  (MatRef(X, trans=True), MatRef(dY), MatRef(dW), 1, K, T, N, Epilogue(accumulate=True), use_f16)]
        outs += [Y, dX, dW]
    return calls, outs


@pytest.mark.parametrize("use_f16", [True, False])
def test_noalloc_matches_the_allocating_entry_point(dev, use_f16):
    for T, seed in ((4096, 21), (1024, 22)):  # the second call smaller than the first
        calls, outs = step_set(dev, T, use_f16, seed)
        init = [o.clone() for o in outs]
        st.matmul_grouped(calls)
        torch.cuda.synchronize()
        want = [o.clone() for o in outs]
        for o, i in zip(outs, init):
            o.copy_(i)
        st.matmul_grouped(calls, noalloc=True)
        torch.cuda.synchronize()
        for i, (o, w) in enumerate(zip(outs, want)):
            assert torch.equal(o, w), (T, i)
        # the product itself, not just agreement: the accumulated dW of the first layer
        X, dY = calls[0][0].h, calls[1][0].h
        ref = (X.double().t() @ dY.double()).float() + 7.0
        if not use_f16:
            assert (outs[2] - ref).abs().max().item() <= 1e-5 * ref.abs().max().item()


def test_noalloc_refuses_partials_beyond_its_scratch(dev):
    """A group whose f32 split-k partials (with column sums) need more than ST_NOALLOC_SCRATCH_BYTES: a wide
    GEMM makes the group use 256-row tiles, and a 256 x 131072 x 1024 GEMM with column sums then splits k 64 ways
    (64 MiB of partials plus 256 KiB of column-sum partials)."""
    big_a, big_b, big_o = (torch.zeros(s, device=dev) for s in ((4096, 128), (128, 4096), (4096, 4096)))
    a = torch.zeros(256, 131072, device=dev)
    b = torch.zeros(131072, 1024, device=dev)
    out = torch.zeros(256 * 1024 + 1024, device=dev)
    calls = [(MatRef(big_a), MatRef(big_b), MatRef(big_o), 1, 4096, 128, 4096, None, False),
             (MatRef(a), MatRef(b), MatRef(out), 1, 256, 131072, 1024,
              Epilogue(col_sum=(256 * 1024, 0)), False)]
    out.fill_(3.0)
    with pytest.raises(st.ScratchtapeError) as e:
        st.matmul_grouped(calls, noalloc=True)
    assert e.value.status == -1 and "fixed scratch" in str(e.value), str(e.value)
    torch.cuda.synchronize()
    assert bool((out == 3.0).all()), "a refused call must launch nothing"


def test_noalloc_refusal_launches_no_group(dev):
    """Two route groups, of which only the second's split-k partials exceed the fixed scratch: an f16 GEMM that
    accumulates into its output (128-row tiles, the first launch of the call) and the f32 group above (256-row
    tiles).  The call is refused before its first launch, so the f16 output keeps its values."""
    big_a, big_b, big_o = (torch.zeros(s, device=dev) for s in ((4096, 128), (128, 4096), (4096, 4096)))
    a = torch.zeros(256, 131072, device=dev)
    b = torch.zeros(131072, 1024, device=dev)
    out = torch.zeros(256 * 1024 + 1024, device=dev)
    x = torch.ones(128, 256, device=dev)
    w = torch.ones(256, 128, device=dev)
    y = torch.full((128, 128), 3.0, device=dev)
    calls = [(MatRef(x), MatRef(w), MatRef(y), 1, 128, 256, 128, Epilogue(accumulate=True), True),
             (MatRef(big_a), MatRef(big_b), MatRef(big_o), 1, 4096, 128, 4096, None, False),
             (MatRef(a), MatRef(b), MatRef(out), 1, 256, 131072, 1024, Epilogue(col_sum=(256 * 1024, 0)), False)]
    with pytest.raises(st.ScratchtapeError) as e:
        st.matmul_grouped(calls, noalloc=True)
    assert e.value.status == -1 and "fixed scratch" in str(e.value), str(e.value)
    torch.cuda.synchronize()
    assert bool((y == 3.0).all()), "the f16 group ran before the refusal"
    # without the oversized GEMM the same call runs: 3 + 256 in every element
    st.matmul_grouped(calls[:2], noalloc=True)
    torch.cuda.synchronize()
    assert bool((y == 259.0).all())
