"""How far the exact integer contract of the 2-bit kNN path ranks from the reference's own f16 scoring and from float64.

The library (and the oracle it is checked against) ranks keys by the exact distance between the query, quantised to
int16 digits with a power-of-two scale, and the dequantised 2-bit key; the reference scores f16(query) against
f16(dequantised key) with matrix cores and a stored f16 norm (ivf.rs:470, 295-300; knn.rs:216), and picks probes
from f16 centroid dots (ivf.rs:62-67, 131-161).  These functions measure, on workloads shaped like the benchmark
(N(0,1) keys in cells of ~10,172 keys, 8 probed cells per query, top-128; 12,288 N(0,1) centroids, 8 probes), the
overlap of the top-k sets each ranking picks:

- `scan_fidelity`: ours vs the reference's f16 scoring, ours vs float64, reference vs float64, where float64 is the
  exact distance between the f32 query and the dequantised key (what both rankings approximate);
- `probe_fidelity`: probe sets, ours vs float64 distances between the f32 query and the f32 centroid, and the
  reference's f16 probe ranking vs the same float64.

Run as a script for the benchmark-size figures (256 queries).
"""
import sys

import numpy as np

import oracle

D = 256
CELL_KEYS = 10_172  # 125,000,000 keys / 12,288 cells
NCELLS = 16  # distinct cells to draw probes from (cells of N(0,1) keys are exchangeable)


def _overlap(a, b):
    """Mean and minimum over rows of |set(a[i]) & set(b[i])| / k, and the fraction of rows with equal sets."""
    k = a.shape[1]
    o = np.array([len(set(x.tolist()) & set(y.tolist())) / k for x, y in zip(a, b)])
    return dict(mean=float(o.mean()), min=float(o.min()), same_set=float((o == 1.0).mean()))


def _topk(dist, ids, k):
    """The k smallest by (dist, id)."""
    order = np.lexsort((ids, dist))[:k]
    return ids[order]


def scan_fidelity(nq, seed=7, k=128, nprobe=8, threads=8):
    rng = np.random.default_rng(seed)
    n = NCELLS * CELL_KEYS
    keys = rng.standard_normal((n, D)).astype(np.float32)
    with oracle.threads(threads):
        codes, scales, norms = oracle.quantize_2bit(keys, D, with_norm=True)
    del keys
    cell_start = np.arange(NCELLS + 1, dtype=np.int64) * CELL_KEYS
    queries = rng.standard_normal((nq, D)).astype(np.float32)
    probes = np.stack([rng.choice(NCELLS, nprobe, replace=False) for _ in range(nq)]).astype(np.int32)

    with oracle.threads(threads):
        ours, _ = oracle.knn_search(codes, scales, cell_start, queries, probes, k)

    # float64: |q - k^|^2 up to the query's own norm, k^ = (u - 1.5) s exactly.
    c = codes.reshape(n, D // 4)
    u = np.stack([(c >> (2 * j)) & 3 for j in range(4)], axis=-1).reshape(n, D).astype(np.float64)
    khat = (u - 1.5) * scales[:, None].astype(np.float64)
    del u
    knorm = (khat * khat).sum(1)
    dots = khat @ queries.astype(np.float64).T  # [n, nq]
    del khat

    ref = np.empty((nq, k), np.int64)
    f64 = np.empty((nq, k), np.int64)
    with oracle.threads(threads):
        for i in range(nq):
            ids = np.concatenate([np.arange(cell_start[p], cell_start[p + 1]) for p in probes[i]])
            rd = np.concatenate([oracle.knn_ref_f16_dists(codes, scales, norms, cell_start[p], cell_start[p + 1],
                                                          queries[i]) for p in probes[i]])
            ref[i] = _topk(rd, ids, k)
            f64[i] = _topk(knorm[ids] - 2.0 * dots[ids, i], ids, k)
    return dict(ours_vs_ref_f16=_overlap(ours, ref), ours_vs_f64=_overlap(ours, f64), ref_f16_vs_f64=_overlap(ref, f64),
                nq=nq, k=k, nprobe=nprobe, cell_keys=CELL_KEYS)


def probe_fidelity(nq, seed=11, nlist=12_288, nprobe=8, threads=8):
    rng = np.random.default_rng(seed)
    cent = rng.standard_normal((nlist, D)).astype(np.float32)
    queries = rng.standard_normal((nq, D)).astype(np.float32)
    ours = oracle.knn_probe(cent, queries, nprobe)
    with oracle.threads(threads):
        ref = oracle.knn_ref_f16_probe(cent, queries, nprobe)
    c64 = cent.astype(np.float64)
    dd = (c64 * c64).sum(1)[None, :] - 2.0 * (queries.astype(np.float64) @ c64.T)
    f64 = np.argsort(dd, axis=1, kind="stable")[:, :nprobe]
    same_order = float((ours == f64).all(1).mean())
    return dict(ours_vs_f64=dict(_overlap(ours, f64), same_order=same_order),
                ref_f16_vs_f64=dict(_overlap(ref, f64), same_order=float((ref == f64).all(1).mean())),
                ours_vs_ref_f16=_overlap(ours, ref), nq=nq, nlist=nlist, nprobe=nprobe)


if __name__ == "__main__":
    import json
    nq = int(sys.argv[1]) if len(sys.argv) > 1 else 256
    print(json.dumps(dict(scan=scan_fidelity(nq), probe=probe_fidelity(nq)), indent=1))
