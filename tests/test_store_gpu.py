"""The 2-bit store on disk in the reference's KnnStore cache format (gpu_step/knn/cache.rs):
the per-key norms bit-exact against the oracle, a save -> load round trip of codes,
scales, cells, values and centroids, and the file's layout read back field by field in
the order cache.rs writes it."""
import struct

import numpy as np
import pytest
import torch

import oracle
from scratchtape_amd import knn, store as st_store

pytestmark = pytest.mark.gpu
D = 256


def make(dev, seed=61):
    rng = np.random.default_rng(seed)
    sizes = rng.integers(0, 900, 9)
    sizes[4] = 0  # an empty cell
    cs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    keys = rng.standard_normal((int(cs[-1]), D)).astype(np.float32)
    s = knn.KnnStore2bit.from_keys(torch.from_numpy(keys).to(dev), cs)
    cent = rng.standard_normal((9, D)).astype(np.float32)
    vals = rng.integers(0, 512, int(cs[-1])).astype(np.float32)
    return s, keys, cs, cent, vals


def test_key_norms_match_the_oracle(dev):
    s, keys, _, _, _ = make(dev)
    wc, ws, want = oracle.quantize_2bit(keys, D, with_norm=True)
    codes, scales = s.codes.cpu().numpy(), s.scales.cpu().numpy()
    bad = np.nonzero((codes != wc).any(1) | (scales != ws))[0]
    assert bad.size == 0, f"quantiser differs on rows {bad[:10]}: scales {scales[bad[:3]]} vs {ws[bad[:3]]}"
    np.testing.assert_array_equal(st_store.key_norms(s.codes, s.scales).cpu().numpy(), want)


def test_save_load_round_trip(dev, tmp_path):
    s, keys, cs, cent, vals = make(dev)
    path = str(tmp_path / "mem.bin")
    st_store.save(path, s, "model-x k=128", extra=77, tile=1024, values=vals, centroids=cent)
    got = st_store.load(path, "model-x k=128", dev)
    assert got is not None and got.extra == 77 and got.tile == 1024
    np.testing.assert_array_equal(got.store.codes.cpu().numpy(), s.codes.cpu().numpy())
    np.testing.assert_array_equal(got.store.scales.cpu().numpy(), s.scales.cpu().numpy())
    np.testing.assert_array_equal(got.store.cell_start, cs)
    np.testing.assert_array_equal(got.values, vals)
    np.testing.assert_array_equal(got.norms, oracle.quantize_2bit(keys, D, with_norm=True)[2])
    np.testing.assert_array_equal(got.centroids, cent.astype(np.float16).astype(np.float32))
    # The reloaded store searches as the original does.
    q = torch.from_numpy(np.random.default_rng(5).standard_normal((6, D)).astype(np.float32)).to(dev)
    p = torch.from_numpy(np.array([[0, 3, 8]] * 6, np.int32)).to(dev)
    a, b = s.search_ivf(q, p), got.store.search_ivf(q, p)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    assert got.store.centroids is not None
    assert st_store.load(path, "another key", dev) is None
    assert st_store.load(str(tmp_path / "missing.bin"), "model-x k=128", dev) is None


def test_file_layout_follows_cache_rs(dev, tmp_path):
    s, keys, cs, cent, vals = make(dev, seed=62)
    path = str(tmp_path / "mem.bin")
    tile = 1024
    st_store.save(path, s, "k", extra=5, tile=tile, values=vals, centroids=cent)
    b = open(path, "rb").read()
    pos = 0

    def u64():
        nonlocal pos
        v = struct.unpack_from("<Q", b, pos)[0]
        pos += 8
        return v

    def blob():
        nonlocal pos
        n = u64()
        out = b[pos:pos + n]
        pos += n
        return out

    n = int(cs[-1])
    assert u64() == 0x5343_5254_4B4E_4E02 and blob() == b"k"
    assert [u64() for _ in range(6)] == [5, D, tile, 1, 2, -(-n // tile)]
    codes, scales = s.codes.cpu().numpy(), s.scales.cpu().numpy()
    _, _, norms = oracle.quantize_2bit(keys, D, with_norm=True)
    for t in range(-(-n // tile)):
        a, e = t * tile, min(n, (t + 1) * tile)
        ln, rp = e - a, -(-(e - a) // 16) * 16
        assert u64() == ln
        kb_ = np.frombuffer(blob(), np.uint8).reshape(rp, D // 4)
        np.testing.assert_array_equal(kb_[:ln], codes[a:e])
        assert not kb_[ln:].any()
        sb = np.frombuffer(blob(), np.float32)
        assert sb.size == rp and np.array_equal(sb[:ln], scales[a:e]) and not sb[ln:].any()
        np.testing.assert_array_equal(np.frombuffer(blob(), np.float32), norms[a:e])
        np.testing.assert_array_equal(np.frombuffer(blob(), np.float32), vals[a:e])
    assert blob() == b""
    assert u64() == 1 and u64() == 9 and u64() == n
    c16 = np.frombuffer(blob(), np.float16)
    assert c16.size == 16 * D and np.array_equal(c16[:9 * D], cent.astype(np.float16).reshape(-1))
    h = cent.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(np.frombuffer(blob(), np.float32), np.cumsum(h * h, 1, dtype=np.float32)[:, -1])
    for c in range(9):
        pieces = [tuple(u64() for _ in range(4)) for _ in range(u64())]
        rows = [g0 + j for (_, a, e, g0) in pieces for j in range(e - a)]
        assert rows == list(range(cs[c], cs[c + 1]))
        for (t, a, e, g0) in pieces:
            assert 0 <= a < e <= tile and g0 == t * tile + a
    assert pos == len(b)
