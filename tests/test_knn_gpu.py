"""2-bit kNN memory on the GPU against the CPU oracle: quantiser bit-exact, and the
IVF scan's per-query top-k index sets (and distances) bit-exact, ties broken by
key index, from small edge cases up to the full 125M-key store."""
import numpy as np
import pytest
import torch

import oracle
from scratchtape_amd import knn

pytestmark = pytest.mark.gpu
D = 256


def test_quantizer_is_bit_exact(dev):
    rng = np.random.default_rng(1)
    keys = rng.standard_normal((5000, D)).astype(np.float32)
    keys[0] = 0.0                      # scale floor 1e-30
    keys[1] *= 1e-20                   # tiny
    keys[2] *= 1e10                    # huge
    keys[3, :] = 0.75 * np.tile([1, -1], D // 2)  # codes 3/0 exactly
    keys[4] = np.where(np.arange(D) < 3, 100.0, 0.001)  # clamping
    codes, scales = knn.quantize_2bit(torch.from_numpy(keys).to(dev))
    wc, ws = oracle.quantize_2bit(keys, D)
    np.testing.assert_array_equal(codes.cpu().numpy(), wc)
    np.testing.assert_array_equal(scales.cpu().numpy(), ws)


def test_synthetic_store_is_the_quantised_synthetic_keys(dev):
    n, row0, seed = 3000, 123_456_789, 7
    keys = knn.synth_keys_f32(seed, row0, n, D, device=dev)
    codes = torch.empty((n, D // 4), dtype=torch.uint8, device=dev)
    scales = torch.empty(n, dtype=torch.float32, device=dev)
    knn.synth_store_2bit(seed, row0, codes, scales)
    k = keys.cpu().numpy()
    assert abs(k.mean()) < 0.01 and abs(k.var() - 1) < 0.01
    wc, ws = oracle.quantize_2bit(k, D)
    np.testing.assert_array_equal(codes.cpu().numpy(), wc)
    np.testing.assert_array_equal(scales.cpu().numpy(), ws)


@pytest.fixture(params=[1, 2], ids=["query_major", "cell_major"])
def scan_order(request):
    """Runs a search test with each scan order of st_knn_search_ivf_2bit (one workgroup per query; each probed cell
    read once for up to four queries): both must give the oracle's results."""
    knn.set_scan_order(request.param)
    yield request.param
    knn.set_scan_order(0)


def make_store(dev, sizes, seed):
    cell_start = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    keys = np.random.default_rng(seed).standard_normal((int(cell_start[-1]), D)).astype(np.float32)
    store = knn.KnnStore2bit.from_keys(torch.from_numpy(keys).to(dev), cell_start)
    return store, store.codes.cpu().numpy(), store.scales.cpu().numpy(), cell_start


def check_search(dev, store, codes, scales, cell_start, queries, probes, k):
    idx, dist = store.search_ivf(torch.from_numpy(queries).to(dev), torch.from_numpy(probes).to(dev), k)
    widx, wdist = oracle.knn_search(codes, scales, cell_start, queries, probes, k)
    np.testing.assert_array_equal(idx.cpu().numpy(), widx)
    np.testing.assert_array_equal(dist.cpu().numpy(), wdist)
    return widx


@pytest.mark.usefixtures("scan_order")
def test_search_small_with_edge_cases(dev):
    rng = np.random.default_rng(2)
    ncells = 40
    sizes = rng.integers(0, 3000, ncells)
    sizes[0], sizes[1], sizes[2] = 0, 3, 1000  # empty cell, tiny cell
    store, codes, scales, cs = make_store(dev, sizes, 3)
    nq = 64
    queries = rng.standard_normal((nq, D)).astype(np.float32)
    queries[0] = 0.0  # zero query: qs = 1, every Q is 0
    queries[1] *= 1e6
    probes = np.stack([rng.choice(ncells, 8, replace=False) for _ in range(nq)]).astype(np.int32)
    probes[2] = [0, 1, 0, 1, 0, 1, 0, 1]  # three keys in total: padding
    probes[3, 5] = probes[3, 1]          # a repeated cell is scanned once
    for k in (128, 10, 1):
        widx = check_search(dev, store, codes, scales, cs, queries, probes, k)
    idx, dist = store.search_ivf(torch.from_numpy(queries).to(dev), torch.from_numpy(probes).to(dev), 128)
    idx = idx.cpu().numpy()
    assert sorted(idx[2][:3]) == [0 + sizes[0], 1 + sizes[0], 2 + sizes[0]] and np.all(idx[2][3:] == -1)


@pytest.mark.usefixtures("scan_order")
@pytest.mark.parametrize("sizes", [[1], [0, 37], [20, 0, 43], [64], [30, 35], [1, 128, 1], [64, 64, 2]])
def test_search_stores_near_one_chunk(dev, sizes):
    # Stores of fewer than 64 keys are read key by key; from 64 keys on, a
    # chunk is read as the 64 keys that end at the store's last row when it
    # would run past it.  Both sides of that boundary, every cell probed.
    rng = np.random.default_rng(len(sizes) * 100 + sum(sizes))
    sizes = np.array(sizes)
    store, codes, scales, cs = make_store(dev, sizes, 13)
    nq, ncells = 5, len(sizes)
    queries = rng.standard_normal((nq, D)).astype(np.float32)
    probes = np.stack([rng.permutation(ncells) for _ in range(nq)]).astype(np.int32)
    for k in (128, 3):
        check_search(dev, store, codes, scales, cs, queries, probes, k)


@pytest.mark.usefixtures("scan_order")
def test_search_many_cells_and_sixteen_probes(dev):
    # 20000 cells of 0..4 keys, 16 probes (the most a query may have), one repeated.
    rng = np.random.default_rng(21)
    ncells = 20000
    sizes = rng.integers(0, 5, ncells)
    store, codes, scales, cs = make_store(dev, sizes, 23)
    nq = 24
    queries = rng.standard_normal((nq, D)).astype(np.float32)
    probes = np.stack([rng.choice(ncells, 16, replace=False) for _ in range(nq)]).astype(np.int32)
    probes[0, 3] = probes[0, 9]
    for k in (128, 5):
        check_search(dev, store, codes, scales, cs, queries, probes, k)


@pytest.mark.usefixtures("scan_order")
def test_search_skips_probe_ids_outside_the_cells(dev):
    # A probe id < 0 or >= ncells is skipped (the header's contract).  The oracle sees each row with those ids
    # replaced by a repeat of one of its valid ids (a repeated cell is scanned once), or, for a row with none, by
    # an empty cell.
    rng = np.random.default_rng(41)
    ncells = 50
    sizes = rng.integers(50, 400, ncells)
    sizes[7] = 0
    store, codes, scales, cs = make_store(dev, sizes, 43)
    nq = 12
    queries = rng.standard_normal((nq, D)).astype(np.float32)
    probes = np.stack([rng.choice(ncells, 8, replace=False) for _ in range(nq)]).astype(np.int32)
    probes[0, 2] = -1
    probes[1, 0] = ncells
    probes[1, 5] = 1 << 30
    probes[2, :] = -1
    probes[3, ::2] = -7
    seen = probes.copy()
    for row in seen:
        valid = [c for c in row if 0 <= c < ncells]
        row[(row < 0) | (row >= ncells)] = valid[0] if valid else 7
    idx, dist = store.search_ivf(torch.from_numpy(queries).to(dev), torch.from_numpy(probes).to(dev), 128)
    widx, wdist = oracle.knn_search(codes, scales, cs, queries, seen, 128)
    np.testing.assert_array_equal(idx.cpu().numpy(), widx)
    np.testing.assert_array_equal(dist.cpu().numpy(), wdist)
    assert np.all(idx.cpu().numpy()[2] == -1)


@pytest.mark.usefixtures("scan_order")
def test_search_random_stores(dev):
    # Seeded random stores (cells of up to 5, 100 or 3000 keys, empty ones included), query
    # magnitudes 2^-20 .. 2^20, probe lists with repeats, nprobe 1..16 and several k.
    rng = np.random.default_rng(47)
    for _ in range(6):
        ncells = int(rng.integers(1, 400))
        sizes = rng.integers(0, int(rng.choice([5, 100, 3000])), ncells)
        store, codes, scales, cs = make_store(dev, sizes, int(rng.integers(1 << 30)))
        nq = int(rng.integers(1, 200))
        nprobe = int(rng.integers(1, min(16, ncells) + 1))
        queries = (rng.standard_normal((nq, D)) * np.exp2(rng.integers(-20, 21, (nq, 1)))).astype(np.float32)
        probes = rng.integers(0, ncells, (nq, nprobe)).astype(np.int32)
        check_search(dev, store, codes, scales, cs, queries, probes, int(rng.choice([1, 7, 64, 128])))


@pytest.mark.usefixtures("scan_order")
def test_search_many_queries_sharing_cells(dev):
    # 600 queries x 8 probes over 100 cells: every cell is probed by ~48 queries.
    rng = np.random.default_rng(31)
    ncells = 100
    sizes = rng.integers(60, 140, ncells)
    store, codes, scales, cs = make_store(dev, sizes, 33)
    nq = 600
    queries = rng.standard_normal((nq, D)).astype(np.float32)
    probes = np.stack([rng.choice(ncells, 8, replace=False) for _ in range(nq)]).astype(np.int32)
    check_search(dev, store, codes, scales, cs, queries, probes, 128)


@pytest.mark.usefixtures("scan_order")
def test_search_ties_break_by_key_index(dev):
    # Identical keys give identical scores: the kept ones must be the lowest indices.
    base = np.random.default_rng(4).standard_normal(D).astype(np.float32)
    keys = np.tile(base, (700, 1))
    cs = np.array([0, 300, 700], np.int64)
    store = knn.KnnStore2bit.from_keys(torch.from_numpy(keys).to(dev), cs)
    q = np.random.default_rng(5).standard_normal((2, D)).astype(np.float32)
    probes = np.array([[1, 0], [0, 1]], np.int32)
    idx, _ = store.search_ivf(torch.from_numpy(q).to(dev), torch.from_numpy(probes).to(dev), 128)
    np.testing.assert_array_equal(idx.cpu().numpy(), np.tile(np.arange(128), (2, 1)))


@pytest.mark.usefixtures("scan_order")
def test_search_cells_of_the_benchmark_size(dev):
    # Cells of ~10.2k keys (125M / 12288), 8 probes per query.
    rng = np.random.default_rng(6)
    ncells = 48
    sizes = rng.poisson(10172, ncells)
    store, codes, scales, cs = make_store(dev, sizes, 7)
    nq = 48
    queries = rng.standard_normal((nq, D)).astype(np.float32)
    probes = np.stack([rng.choice(ncells, 8, replace=False) for _ in range(nq)]).astype(np.int32)
    check_search(dev, store, codes, scales, cs, queries, probes, 128)


def test_full_store_125m_keys(dev):
    """The benchmark's store: 125M keys in 12288 cells, 256 queries x 8 probes; every query's top-128 (indices and
    distances) bit-exact against the oracle over the batch's probed cells."""
    n, ncells, nq, nprobe, seed = 125_000_000, 12288, 256, 8, 11
    rng = np.random.default_rng(seed)
    sizes = rng.multinomial(n, np.full(ncells, 1.0 / ncells))
    cs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    codes = torch.empty((n, D // 4), dtype=torch.uint8, device=dev)
    scales = torch.empty(n, dtype=torch.float32, device=dev)
    knn.synth_store_2bit(seed, 0, codes, scales)
    store = knn.KnnStore2bit(codes, scales, cs)
    queries = rng.standard_normal((nq, D)).astype(np.float32)
    probes = np.stack([rng.choice(ncells, nprobe, replace=False) for _ in range(nq)]).astype(np.int32)
    idx, dist = store.search_ivf(torch.from_numpy(queries).to(dev), torch.from_numpy(probes).to(dev), 128)
    idx, dist = idx.cpu().numpy(), dist.cpu().numpy()
    # The oracle scores a compact copy of the batch's distinct probed cells (about 1.3 GB) with every query's
    # probes renumbered into it; its row indices map back through `allrows`.
    cells = np.unique(probes)
    rows = [np.arange(cs[c], cs[c + 1]) for c in cells]
    sub_cs = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int64)
    allrows = np.concatenate(rows)
    sel = torch.from_numpy(allrows).to(dev)
    sc, ss = codes[sel].cpu().numpy(), scales[sel].cpu().numpy()
    del sel
    sub_probes = np.searchsorted(cells, probes).astype(np.int32)
    with oracle.threads(16):
        widx, wdist = oracle.knn_search(sc, ss, sub_cs, queries, sub_probes, 128)
    np.testing.assert_array_equal(idx, np.where(widx >= 0, allrows[np.maximum(widx, 0)], -1))
    np.testing.assert_array_equal(dist, wdist)
    # every result lies in its query's probed cells and is sorted
    assert np.all(np.diff(dist, axis=1) >= 0)
    cell_of = np.searchsorted(cs, idx, side="right") - 1
    assert np.all(np.any(cell_of[:, :, None] == probes[:, None, :], axis=2))
    del codes, scales, store
    torch.cuda.empty_cache()


def test_full_store_2048_queries_cell_major(dev):
    """A large batch on the benchmark's store: 2048 queries x 8 probes over 12288 cells (each cell probed 1.3 times
    on average, so the call takes the cell-major scan by itself); every query's top-128 bit-exact against the oracle
    over the batch's probed cells, and every query also against the query-major scan."""
    n, ncells, nq, nprobe, seed = 125_000_000, 12288, 2048, 8, 12
    rng = np.random.default_rng(seed)
    sizes = rng.multinomial(n, np.full(ncells, 1.0 / ncells))
    cs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    codes = torch.empty((n, D // 4), dtype=torch.uint8, device=dev)
    scales = torch.empty(n, dtype=torch.float32, device=dev)
    knn.synth_store_2bit(seed, 0, codes, scales)
    store = knn.KnnStore2bit(codes, scales, cs)
    queries = rng.standard_normal((nq, D)).astype(np.float32)
    probes = np.stack([rng.choice(ncells, nprobe, replace=False) for _ in range(nq)]).astype(np.int32)
    qd, pd = torch.from_numpy(queries).to(dev), torch.from_numpy(probes).to(dev)
    idx, dist = store.search_ivf(qd, pd, 128)
    idx, dist = idx.cpu().numpy(), dist.cpu().numpy()
    knn.set_scan_order(1)
    try:
        idx1, dist1 = store.search_ivf(qd, pd, 128)
    finally:
        knn.set_scan_order(0)
    np.testing.assert_array_equal(idx, idx1.cpu().numpy())
    np.testing.assert_array_equal(dist, dist1.cpu().numpy())
    # The oracle scores a compact copy of the batch's distinct probed cells with the probes renumbered into it.
    cells = np.unique(probes)
    rows = [np.arange(cs[c], cs[c + 1]) for c in cells]
    sub_cs = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int64)
    allrows = np.concatenate(rows)
    sel = torch.from_numpy(allrows).to(dev)
    sc, ss = codes[sel].cpu().numpy(), scales[sel].cpu().numpy()
    del sel
    sub_probes = np.searchsorted(cells, probes).astype(np.int32)
    with oracle.threads(16):
        widx, wdist = oracle.knn_search(sc, ss, sub_cs, queries, sub_probes, 128)
    np.testing.assert_array_equal(idx, np.where(widx >= 0, allrows[np.maximum(widx, 0)], -1))
    np.testing.assert_array_equal(dist, wdist)
    del codes, scales, store, sc, ss
    torch.cuda.empty_cache()


# --------------------------------------------------------------------------- masked exact search (knn.rs:295-331)


@pytest.mark.parametrize("always,k", [(0, 128), (37, 128), (5000, 10), (20000, 128)])
def test_masked_search_matches_oracle(dev, always, k):
    rng = np.random.default_rng(51)
    n, nq = 20000, 40
    keys = rng.standard_normal((n, D)).astype(np.float32)
    store = knn.KnnStore2bit.from_keys(torch.from_numpy(keys).to(dev), np.array([0, n], np.int64))
    codes, scales = store.codes.cpu().numpy(), store.scales.cpu().numpy()
    queries = rng.standard_normal((nq, D)).astype(np.float32)
    lo = rng.integers(0, n, nq)
    hi = lo + rng.integers(0, 6000, nq)  # some past the store's end (clipped)
    lo[0], hi[0] = 300, 300              # empty range: the always prefix only
    lo[1], hi[1] = n - 5, n + 100        # 5 keys
    lo[2], hi[2] = 0, n                  # everything
    lo[3], hi[3] = 64, 128               # one aligned chunk
    lo[4], hi[4] = 10, 5                 # inverted: empty
    queries[5] *= np.float32(2.0 ** -130)  # a subnormal query (exact power-of-two quantisation)
    lohi = torch.from_numpy(np.stack([lo, hi], 1).astype(np.int64)).to(dev)
    idx, dist = store.search_masked(torch.from_numpy(queries).to(dev), lohi, always, k)
    widx, wdist = oracle.knn_search_masked(codes, scales, queries, lo, hi, always, k)
    np.testing.assert_array_equal(idx.cpu().numpy(), widx)
    np.testing.assert_array_equal(dist.cpu().numpy(), wdist)


def test_masked_search_over_a_window_of_the_full_store(dev):
    # The 125M-key store's last 1M keys as the in-document window of 4 queries (search_tail's use).
    n = 125_000_000
    codes = torch.empty((n, D // 4), dtype=torch.uint8, device=dev)
    scales = torch.empty(n, dtype=torch.float32, device=dev)
    knn.synth_store_2bit(2024, 0, codes, scales)
    store = knn.KnnStore2bit(codes, scales, np.array([0, n], np.int64))
    rng = np.random.default_rng(52)
    queries = rng.standard_normal((4, D)).astype(np.float32)
    lo = np.array([n - 1_000_000, n - 700_000, n - 65, n - 1_000_000], np.int64)
    hi = np.array([n, n - 300_000, n, n - 999_000], np.int64)
    lohi = torch.from_numpy(np.stack([lo, hi], 1)).to(dev)
    idx, dist = store.search_masked(torch.from_numpy(queries).to(dev), lohi, 0, 128)
    w0 = int(lo.min())
    sub_codes, sub_scales = codes[w0:].cpu().numpy(), scales[w0:].cpu().numpy()
    widx, wdist = oracle.knn_search_masked(sub_codes, sub_scales, queries, lo - w0, hi - w0, 0, 128)
    np.testing.assert_array_equal(idx.cpu().numpy(), np.where(widx >= 0, widx + w0, -1))
    np.testing.assert_array_equal(dist.cpu().numpy(), wdist)
    del codes, scales
    torch.cuda.empty_cache()
