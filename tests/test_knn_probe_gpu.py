"""IVF probe selection on the GPU against the CPU oracle: the centroid store (digits'
exponents and norms) and each query's nprobe nearest cells, bit-exact, ties to the
lower cell id; then search_ivf by nprobe end to end."""
import numpy as np
import pytest
import torch

import oracle
from scratchtape_amd import knn

pytestmark = pytest.mark.gpu
D = 256


def run_probe(dev, cent, queries, nprobe):
    c = knn.Centroids(torch.from_numpy(cent).to(dev))
    got = c.probe(torch.from_numpy(queries).to(dev), nprobe).cpu().numpy()
    return c, got


def test_centroid_store_matches_the_oracle(dev):
    rng = np.random.default_rng(31)
    cent = rng.standard_normal((61, D)).astype(np.float32)  # 61: a partial last block of 8
    cent[0] = 0.0
    cent[1] *= np.float32(2.0 ** -60)
    cent[2] *= np.float32(2.0 ** 60)
    cent[3] = np.where(np.arange(D) < 2, 1.0, 0.0)  # max at the top of the int16 range
    cent[4] = -cent[3]
    c = knn.Centroids(torch.from_numpy(cent).to(dev))
    _, wexp, wnorm = oracle.knn_centroid_prep(cent)
    np.testing.assert_array_equal(c.cexp.cpu().numpy(), wexp)
    np.testing.assert_array_equal(c.cnorm.cpu().numpy(), wnorm)
    assert c.digits.numel() == 8 * 4096


@pytest.mark.parametrize("nlist,nq,nprobe", [(5, 3, 5), (8, 1, 1), (300, 7, 8), (1000, 130, 16), (1537, 64, 3)])
def test_probe_matches_the_oracle(dev, nlist, nq, nprobe):
    rng = np.random.default_rng(nlist * 7 + nq)
    cent = rng.standard_normal((nlist, D)).astype(np.float32)
    queries = rng.standard_normal((nq, D)).astype(np.float32)
    _, got = run_probe(dev, cent, queries, nprobe)
    np.testing.assert_array_equal(got, oracle.knn_probe(cent, queries, nprobe))


def test_probe_edge_cases(dev):
    rng = np.random.default_rng(32)
    nlist = 200
    cent = rng.standard_normal((nlist, D)).astype(np.float32)
    cent *= np.exp2(rng.integers(-30, 31, nlist)).astype(np.float32)[:, None]  # magnitudes 2^-30 .. 2^30
    cent[10] = 0.0
    cent[77] = cent[12]   # duplicates: equal dd, ties to the lower id
    cent[150] = cent[12]
    queries = rng.standard_normal((40, D)).astype(np.float32)
    queries *= np.exp2(rng.integers(-30, 31, 40)).astype(np.float32)[:, None]
    queries[0] = 0.0                 # ranks by centroid norm
    queries[1] = cent[12]            # the duplicated centroid itself
    queries[2] = cent[33]
    queries[3] = np.float32(1e6) * np.sign(rng.standard_normal(D)).astype(np.float32)
    for nprobe in (1, 4, 16):
        _, got = run_probe(dev, cent, queries, nprobe)
        np.testing.assert_array_equal(got, oracle.knn_probe(cent, queries, nprobe))
    assert list(got[1, :3]) == [12, 77, 150] and got[2, 0] == 33


def test_probe_at_the_benchmark_shape(dev):
    # 12288 cells, 256 queries, 8 probes: the scan benchmark's batch.
    g = torch.Generator(device=dev).manual_seed(5)
    cent = torch.randn((12288, D), generator=g, device=dev)
    queries = torch.randn((256, D), generator=g, device=dev)
    got = knn.Centroids(cent).probe(queries, 8).cpu().numpy()
    np.testing.assert_array_equal(got, oracle.knn_probe(cent.cpu().numpy(), queries.cpu().numpy(), 8))


def test_probe_in_several_query_chunks(dev):
    # 600,000 cells: a dd chunk holds 64 queries, so 130 queries take three chunks.
    g = torch.Generator(device=dev).manual_seed(6)
    nlist = 600_000
    cent = torch.randn((nlist, D), generator=g, device=dev)
    queries = torch.randn((130, D), generator=g, device=dev)
    c = knn.Centroids(cent)
    got = c.probe(queries, 16).cpu().numpy()
    parts = np.concatenate([c.probe(queries[a:b].contiguous(), 16).cpu().numpy() for a, b in ((0, 63), (63, 130))])
    np.testing.assert_array_equal(got, parts)
    sample = [0, 63, 64, 127, 128, 129]  # each side of each chunk boundary, against the oracle
    prep = oracle.knn_centroid_prep(cent.cpu().numpy())
    want = oracle.knn_probe(None, queries.cpu().numpy()[sample], 16, prep=prep)
    np.testing.assert_array_equal(got[sample], want)


def test_search_ivf_by_nprobe_end_to_end(dev):
    rng = np.random.default_rng(33)
    ncells = 48
    sizes = rng.integers(0, 2500, ncells)
    cell_start = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    cent = rng.standard_normal((ncells, D)).astype(np.float32)
    # Keys scattered around their cell's centroid, stored cell-contiguous.
    keys = (np.repeat(cent, sizes, axis=0) + 0.8 * rng.standard_normal((int(cell_start[-1]), D))).astype(np.float32)
    store = knn.KnnStore2bit.from_keys(torch.from_numpy(keys).to(dev), cell_start)
    store.set_centroids(torch.from_numpy(cent).to(dev))
    queries = (cent[rng.integers(0, ncells, 20)] + 0.8 * rng.standard_normal((20, D))).astype(np.float32)
    idx, dist = store.search_ivf(torch.from_numpy(queries).to(dev), 6)
    probes = oracle.knn_probe(cent, queries, 6)
    widx, wdist = oracle.knn_search(store.codes.cpu().numpy(), store.scales.cpu().numpy(), cell_start, queries, probes)
    np.testing.assert_array_equal(idx.cpu().numpy(), widx)
    np.testing.assert_array_equal(dist.cpu().numpy(), wdist)


@pytest.mark.parametrize("case", ["all_equal", "many_equal_nearest", "near_equal_nearest", "one_cell_last_round"])
def test_probe_selection_under_ties_and_round_edges(dev, case):
    # Equal or near-equal distances fill the selection's candidate buffer past one
    # wave (many_equal, near_equal) or past its capacity (all_equal: 3000 candidates);
    # 12289 cells leave one cell for the second round of 12288.
    rng = np.random.default_rng(34)
    nlist = 12289 if case == "one_cell_last_round" else 3000
    cent = rng.standard_normal((nlist, D)).astype(np.float32)
    queries = rng.standard_normal((5, D)).astype(np.float32)
    if case == "all_equal":
        cent[:] = cent[0]
    elif case in ("many_equal_nearest", "near_equal_nearest"):
        idx = rng.choice(nlist, 300, replace=False)
        cent[idx] = queries[0]
        if case == "near_equal_nearest":
            cent[idx] += np.float32(1e-4) * rng.standard_normal((300, D)).astype(np.float32)
    else:
        cent[12288] = queries[1]
    for nprobe in (1, 8, 16):
        _, got = run_probe(dev, cent, queries, nprobe)
        np.testing.assert_array_equal(got, oracle.knn_probe(cent, queries, nprobe))
    if case == "all_equal":
        assert list(got[0]) == list(range(16))
    if case == "one_cell_last_round":
        assert got[1, 0] == 12288


def test_probe_random_indexes(dev):
    # Seeded random indexes: 1..5000 cells, magnitudes 2^-25 .. 2^25 on both sides, duplicated
    # centroids (ties to the lower id), zero queries, nprobe 1..16.
    rng = np.random.default_rng(35)
    for _ in range(8):
        nlist = int(rng.choice([int(rng.integers(1, 100)), int(rng.integers(100, 5000))]))
        nq = int(rng.integers(1, 300))
        nprobe = int(rng.integers(1, min(16, nlist) + 1))
        cent = (rng.standard_normal((nlist, D)) * np.exp2(rng.integers(-25, 26, (nlist, 1)))).astype(np.float32)
        if rng.random() < 0.5:
            cent[rng.integers(0, nlist, max(1, nlist // 10))] = cent[int(rng.integers(0, nlist))]
        queries = (rng.standard_normal((nq, D)) * np.exp2(rng.integers(-25, 26, (nq, 1)))).astype(np.float32)
        queries[0] = 0.0
        _, got = run_probe(dev, cent, queries, nprobe)
        np.testing.assert_array_equal(got, oracle.knn_probe(cent, queries, nprobe))
