"""The timed paths replayed from HIP graphs, as the benchmark runs them: each graph is replayed several times with
the program's own eager work and synchronisations in between, and every replay must give the eager results bit for
bit (the same kernels on the same inputs are deterministic).  Nothing here records a memset into a graph: the
grouped GEMM's split-k sums, the row kernels' partials and every clear are kernels."""
import numpy as np
import pytest
import torch

import scratchtape_amd as st
from scratchtape_amd import MatRef, attention, knn, rows

pytestmark = pytest.mark.gpu

REPLAYS = 3


def replay_and_check(fn, outputs, reset=None):
    """Eager run -> reference copies; then a graph of two calls of fn, replayed REPLAYS times (stale outputs
    cannot pass: they are overwritten with NaN, or -7 for integers, before each replay)."""
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        if reset:
            reset()
        fn()
        torch.cuda.synchronize()
        want = [o.clone() for o in outputs]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            if reset:
                reset()
            fn()
            if reset:
                reset()
            fn()
        junk = torch.randn(1 << 20, device="cuda")
        for r in range(REPLAYS):
            for o in outputs:
                o.fill_(float("nan") if o.is_floating_point() else -7)  # eager work between replays
            junk.mul_(1.0001).add_(0.5)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            for i, (o, w) in enumerate(zip(outputs, want)):
                assert torch.equal(o, w), (r, i)
        del g


def step_set(dev, use_f16, seed=5):
    """The 15 GEMMs of a d_model-256 step at T = 1024 (the dW GEMMs split, so k_sum_group runs)."""
    T, calls, outs = 1024, [], []
    gen = torch.Generator(device="cpu").manual_seed(seed)
    for K, N in [(256, 768), (256, 256), (256, 1024), (1024, 256), (256, 256)]:
        X, W, dY = (torch.randn(s, generator=gen).to(dev) for s in ((T, K), (K, N), (T, N)))
        Y, dX, dW = torch.zeros(T, N, device=dev), torch.zeros(T, K, device=dev), torch.zeros(K, N, device=dev)
        calls += [(MatRef(X), MatRef(W), MatRef(Y), 1, T, K, N, None, use_f16),
                  (MatRef(dY), MatRef(W, trans=True), MatRef(dX), 1, T, N, K, None, use_f16),
                  (MatRef(X, trans=True), MatRef(dY), MatRef(dW), 1, K, T, N, None, use_f16)]
        outs += [Y, dX, dW]
    return calls, outs


@pytest.mark.parametrize("use_f16", [True, False])
def test_grouped_step_set_replays_from_a_graph(dev, use_f16):
    calls, outs = step_set(dev, use_f16)
    replay_and_check(lambda: st.matmul_grouped(calls), outs)


def test_fused_attention_step_replays_from_a_graph(dev):
    b, h, t, hd = 4, 4, 128, 64
    d = h * hd
    gen = torch.Generator(device="cpu").manual_seed(9)
    qkv = torch.randn(b * t * 3 * d, generator=gen).half().float().to(dev)
    dctx = torch.randn(b * t * d, generator=gen).to(dev)
    buf = attention.FusedBuffers.empty(b, h, t, hd, dev)
    replay_and_check(lambda: attention.fused_step(qkv, dctx, buf, b, h, t, hd), [buf.ctx, buf.lse, buf.dqkv])


def test_layer_norm_step_replays_from_a_graph(dev):
    n, d = 1024, 256
    gen = torch.Generator(device="cpu").manual_seed(13)
    x = torch.randn(n * d, generator=gen).to(dev)
    dy = torch.randn(n * d, generator=gen).to(dev)
    params = torch.cat([1 + 0.1 * torch.randn(d, generator=gen), 0.1 * torch.randn(d, generator=gen)]).to(dev)
    grads = torch.zeros(2 * d, device=dev)
    dx = torch.empty(n * d, device=dev)
    box = {}

    def step():
        box["f"] = rows.layer_norm(x, n, d, params, 0, 1e-5)
        rows.layer_norm_backward(dy, x, box["f"], n, d, params, grads, 0, dx, False)

    # the parameter gradients accumulate: cleared (a fill kernel) before each step
    step()
    torch.cuda.synchronize()
    replay_and_check(step, [dx, grads], reset=grads.zero_)


def test_knn_search_probe_and_masked_search_replay_from_a_graph(dev):
    """The benchmark's kNN lines: probe selection, the IVF scan and the masked scan, one graph."""
    rng = np.random.default_rng(17)
    sizes = rng.integers(200, 900, 48)
    cell_start = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    keys = torch.from_numpy(rng.standard_normal((int(cell_start[-1]), 256)).astype(np.float32)).to(dev)
    store = knn.KnnStore2bit.from_keys(keys, cell_start)
    store.set_centroids(torch.from_numpy(rng.standard_normal((48, 256)).astype(np.float32)).to(dev))
    nq = 24
    q = torch.from_numpy(rng.standard_normal((nq, 256)).astype(np.float32)).to(dev)
    probes = torch.empty((nq, 6), dtype=torch.int32, device=dev)
    lo = rng.integers(0, int(cell_start[-1]) - 3000, nq)
    lohi = torch.from_numpy(np.stack([lo, lo + 3000], 1).astype(np.int64)).to(dev)
    ivf = (torch.empty((nq, 128), dtype=torch.int64, device=dev), torch.empty((nq, 128), device=dev))
    msk = (torch.empty((nq, 128), dtype=torch.int64, device=dev), torch.empty((nq, 128), device=dev))

    def step():
        store.centroids.probe(q, 6, out=probes)
        store.search_ivf(q, probes, 128, out=ivf)
        store.search_masked(q, lohi, 500, 128, out=msk)
    replay_and_check(step, [probes, *ivf, *msk])
