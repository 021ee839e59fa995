"""Floors on how closely the exact integer contract of the 2-bit kNN path ranks like the reference's own f16 scoring
and like float64 (knn_fidelity.py measures; ivf.rs:715-826 is the reference's own recall check, whose 2-bit case
allows any ranking, tol = infinity).

Benchmark-size figures (256 queries, `python tests/knn_fidelity.py 256` from the repository root with the root on
PYTHONPATH), top-128 over 8 probed cells of 10,172 N(0,1) keys: ours vs the reference's f16 scoring 0.9973 mean
overlap (min 0.984), ours vs float64 0.9998, the reference's f16 scoring vs float64 0.9975; probe sets over 12,288
N(0,1) centroids: ours equal float64's for every query, the reference's f16 probes for 99.6 %.
"""
import numpy as np
import pytest

import oracle
import knn_fidelity


def test_batched_reference_scoring_equals_the_single_key_restatement():
    d = 256
    rng = np.random.default_rng(5)
    keys = rng.standard_normal((64, d)).astype(np.float32)
    codes, scales, norms = oracle.quantize_2bit(keys, d, with_norm=True)
    q = rng.standard_normal(d).astype(np.float32)
    got = oracle.knn_ref_f16_dists(codes, scales, norms, 8, 40, q)
    want = np.array([oracle.knn_ref_f16_dist(codes[r], scales[r], norms[r], q) for r in range(8, 40)], np.float32)
    assert np.array_equal(got, want)


def _f16(x):
    return np.float32(np.float16(x))


def test_reference_probe_ranking_on_a_hand_sized_case():
    """orc_knn_ref_f16_probe against a scalar loop of the same rules (f16 operands, f32 sums in index order,
    dd = cnorm - 2 dot, strict < insertion)."""
    rng = np.random.default_rng(9)
    nlist, d, nq, nprobe = 40, 16, 5, 4
    cent = rng.standard_normal((nlist, d)).astype(np.float32)
    cent[7] = cent[3]  # an exact tie: the lower cell must come first
    queries = rng.standard_normal((nq, d)).astype(np.float32)
    queries[0] = cent[3] * np.float32(1.0001)
    got = oracle.knn_ref_f16_probe(cent, queries, nprobe)
    for i in range(nq):
        dd = []
        for c in range(nlist):
            norm, dot = np.float32(0), np.float32(0)
            for j in range(d):
                x = _f16(cent[c, j])
                norm = np.float32(norm + x * x)
                dot = np.float32(dot + _f16(queries[i, j]) * x)
            dd.append(np.float32(norm - np.float32(2) * dot))
        want = sorted(range(nlist), key=lambda c: (dd[c], c))[:nprobe]
        assert got[i].tolist() == want, i
    assert got[0][:2].tolist() == [3, 7]


def test_scan_top128_overlap_floors():
    r = knn_fidelity.scan_fidelity(32)
    # The exact contract agrees with float64 almost everywhere, and with the reference's f16 scoring as closely
    # as the reference agrees with float64 itself.
    assert r["ours_vs_f64"]["mean"] >= 0.999 and r["ours_vs_f64"]["min"] >= 0.99, r
    assert r["ours_vs_ref_f16"]["mean"] >= 0.99 and r["ours_vs_ref_f16"]["min"] >= 0.96, r
    assert r["ours_vs_f64"]["mean"] >= r["ref_f16_vs_f64"]["mean"], r


def test_probe_set_agreement_floors():
    r = knn_fidelity.probe_fidelity(64)
    assert r["ours_vs_f64"]["same_set"] >= 0.98 and r["ours_vs_f64"]["mean"] >= 0.995, r
    assert r["ours_vs_ref_f16"]["mean"] >= 0.99, r
    assert r["ours_vs_f64"]["mean"] >= r["ref_f16_vs_f64"]["mean"], r


@pytest.mark.parametrize("planted", ["one_term", "sign"])
def test_the_overlap_measure_sees_a_planted_ranking_mistake(planted):
    """A ranking with a dropped or sign-flipped term overlaps float64's far less: the floors are not vacuous."""
    rng = np.random.default_rng(3)
    n, nq, k = 4000, 8, 128
    keys = rng.standard_normal((n, 256))
    q = rng.standard_normal((nq, 256))
    knorm = (keys * keys).sum(1)
    good = np.stack([np.argsort(knorm - 2 * keys @ qi, kind="stable")[:k] for qi in q])
    bad_d = [(-2 * keys @ qi) if planted == "one_term" else (knorm + 2 * keys @ qi) for qi in q]
    bad = np.stack([np.argsort(b, kind="stable")[:k] for b in bad_d])
    assert knn_fidelity._overlap(good, good)["mean"] == 1.0
    assert knn_fidelity._overlap(bad, good)["mean"] < 0.9
