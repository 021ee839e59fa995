"""The library's scratch memory under HIP graphs and host threads.

- A split-k GEMM captured into a graph keeps working after a larger eager split-k GEMM grew the arena: the buffer the
  graph holds is kept (not freed) until st_scratch_release.
- Growing the arena while the stream is being captured is refused with a message, and nothing is launched.
- st_ndarray_matmul (NdArray::matmul, tensor.rs:241) called from several host threads at once on a shape that splits
  k gives each thread the oracle's product: each call has its own scratch.
"""
import threading

import numpy as np
import pytest
import torch

import oracle
import scratchtape_amd as st
from scratchtape_amd import MatRef
from scratchtape_amd.tensor import ndarray_matmul

pytestmark = pytest.mark.gpu


def split_gemm(dev, m, k, n, seed):
    """out = a @ b with few output tiles and a long k, which the GEMM splits over k (scratch partials)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    a = torch.randn(m, k, generator=g).to(dev)
    b = torch.randn(k, n, generator=g).to(dev)
    out = torch.zeros(m, n, device=dev)
    return a, b, out, (lambda: st.matmul_f32(MatRef(a), MatRef(b), MatRef(out), 1, m, k, n))


def test_graph_replays_after_the_arena_grew(dev):
    st.lib().st_scratch_release()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        a, b, out, small = split_gemm(dev, 256, 4096, 256, 1)
        small()
        torch.cuda.synchronize()
        want = out.clone()
        ref = (a.double() @ b.double()).float()
        assert (want - ref).abs().max().item() <= 1e-5 * ref.abs().max().item()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            small()
        # A larger split-k GEMM grows the arena (4x the partials); the graph's buffer must survive it.
        a2, b2, out2, big = split_gemm(dev, 512, 8192, 512, 2)
        big()
        torch.cuda.synchronize()
        ref2 = (a2.double() @ b2.double()).float()
        assert (out2 - ref2).abs().max().item() <= 1e-5 * ref2.abs().max().item()
        for _ in range(3):
            out.fill_(float("nan"))
            big()  # eager work on the new arena between replays
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, want)
        del g
    torch.cuda.synchronize()
    assert st.lib().st_scratch_release() == 0


def test_growth_during_capture_is_refused(dev):
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        a, b, out, call = split_gemm(dev, 256, 4096, 256, 3)
        call()  # device checks done outside the capture
        torch.cuda.synchronize()
        st.lib().st_scratch_release()  # the next split-k call has to allocate
        out.fill_(-1.0)
        g = torch.cuda.CUDAGraph()
        err = None
        with torch.cuda.graph(g, stream=s):
            try:
                call()
            except st.ScratchtapeError as e:
                err = e
        assert err is not None and err.status == -1, err
        assert "captured" in str(err) and "before capturing" in str(err), str(err)
        del g
        torch.cuda.synchronize()
        assert bool((out == -1.0).all()), "a refused call must launch nothing"
        call()  # outside capture the arena grows again
        torch.cuda.synchronize()
        ref = (a.double() @ b.double()).float()
        assert (out - ref).abs().max().item() <= 1e-5 * ref.abs().max().item()


def test_ndarray_matmul_from_several_threads(dev):
    m, k, n = 256, 4096, 256
    rng = np.random.default_rng(11)
    inputs = [(rng.uniform(-1, 1, (m, k)).astype(np.float32), rng.uniform(-1, 1, (k, n)).astype(np.float32))
              for _ in range(4)]
    results = [None] * 4
    errors = []

    def work(i):
        try:
            for _ in range(3):
                results[i] = ndarray_matmul(*inputs[i])
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for (a, b), got in zip(inputs, results):
        want = oracle.matmul(a, b)
        assert float(np.max(np.abs(got - want))) <= 1e-5 * float(np.max(np.abs(want)))
