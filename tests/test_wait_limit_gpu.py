"""The grouped f16 GEMM kernel's bounded slot waits: a wait that gives up is reported, not silent.

Its producer and consumer waves hand LDS slots over through counters, and each wait polls a bounded number of
times so that every wave always ends.  The host sets the bound to 0 here, so the first wait of every consumer
gives up (its producers cannot have filled the slot before the first poll): the kernel still runs to its end,
every wave exits normally, and st_sync reports the give-ups as an error (the reference's failures are panics,
tensor.rs:253, gpu_step/matmul.rs:107).  With the default bound the same call is checked again and is exact."""
import pytest
import torch

import scratchtape_amd as st
from scratchtape_amd import MatRef

pytestmark = pytest.mark.gpu


def _group(dev):
    gen = torch.Generator(device="cpu").manual_seed(5)
    X = torch.randn(1024, 256, generator=gen).to(dev)
    W = torch.randn(256, 512, generator=gen).to(dev)
    Y = torch.zeros(1024, 512, device=dev)
    return X, W, Y, [(MatRef(X), MatRef(W), MatRef(Y), 1, 1024, 256, 512, None, True)]


def test_a_wait_that_gives_up_is_reported(dev):
    X, W, Y, calls = _group(dev)
    st.sync()  # nothing pending from earlier tests
    try:
        st.set_wait_limit(0)
        st.matmul_grouped(calls)
        with pytest.raises(st.ScratchtapeError) as e:
            st.sync()
        assert e.value.status == -2 and "gave up" in str(e.value), str(e.value)
    finally:
        st.set_wait_limit(-1)
    # the count was cleared by the report; with the default bound the call is exact again
    st.sync()
    Y.zero_()
    st.matmul_grouped(calls)
    st.sync()
    want = X.half().double() @ W.half().double()
    err = ((Y.double() - want).abs().max() / want.abs().max()).item()
    assert err <= 1e-5, err
