"""2-bit kNN memory on MI355X: the store, its device quantiser and the scored IVF search.

Mirrors the quantised `KnnStore` (gpu_step/knn.rs:57-236) and the scored part of
`KnnStore::search_ivf` (gpu_step/knn/ivf.rs:466-686) for 2-bit keys of width
256: keys live cell-contiguous on the device (as `build_ivf` reorders them,
ivf.rs:386-432), one f32 scale per key, codes packed 4 per byte.  The search
takes each query's probed cells and returns, per query, the k nearest keys by
the exact 2-bit score, ascending by (distance, key index), as global row
indices with distances max(|q^|^2 + dist, 0) (ivf.rs:673-684).

Probe selection (ivf.rs:62-69 `Cent`, ivf.rs:128-161 `k_probe`, the probe stage
of `search_ivf` ivf.rs:473-489) runs on the device too: `Centroids` holds the
quantised centroids, and `search_ivf(queries, nprobe)` picks each query's
nprobe nearest cells by the exact integer distance before scanning them.
`search_masked` is the store's masked exact search (knn.rs:295-331): each query
scores the keys of its own (lo, hi) range plus an always-visible prefix.
"""
from __future__ import annotations

from typing import Optional, Tuple

import numpy as np
import torch

from . import _lib
from .matmul import _stream

KMAX = 128      # knn.rs:21
PROBE_MAX = 16  # ivf.rs:126


def _dptr(t: torch.Tensor, dtype: torch.dtype, what: str) -> int:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{what} must be a GPU tensor")
    if t.dtype != dtype or not t.is_contiguous():
        raise ValueError(f"{what} must be a contiguous {dtype} tensor")
    return t.data_ptr()


def quantize_2bit(keys: torch.Tensor, stream=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """tile_of for 2-bit keys (knn.rs:190-225) on the device: keys [n, d] -> (codes [n, d/4] u8, scales [n])."""
    n, d = keys.shape
    codes = torch.empty((n, d // 4), dtype=torch.uint8, device=keys.device)
    scales = torch.empty(n, dtype=torch.float32, device=keys.device)
    _lib.call("st_knn_quantize_2bit", _dptr(keys, torch.float32, "keys"), n, d, codes.data_ptr(),
              scales.data_ptr(), _stream(stream))
    return codes, scales


def synth_store_2bit(seed: int, row0: int, codes: torch.Tensor, scales: torch.Tensor, stream=None) -> None:
    """Fills codes/scales (rows row0.. of a synthetic store) with quantised N(0,1) keys (benchmark support)."""
    n, kb = codes.shape
    _lib.call("st_knn_synth_store_2bit", seed, row0, n, kb * 4, _dptr(codes, torch.uint8, "codes"),
              _dptr(scales, torch.float32, "scales"), _stream(stream))


def synth_keys_f32(seed: int, row0: int, n: int, d: int = 256, device="cuda", stream=None) -> torch.Tensor:
    """The f32 keys synth_store_2bit quantises for rows row0..row0+n."""
    keys = torch.empty((n, d), dtype=torch.float32, device=device)
    _lib.call("st_knn_synth_keys_f32", seed, row0, n, d, keys.data_ptr(), _stream(stream))
    return keys


def set_scan_order(order: int) -> None:
    """st_knn_set_scan_order: how search_ivf scans, process-wide (0 chooses by batch size, 1 a workgroup per query,
    2 each probed cell once for up to four queries)."""
    _lib.call("st_knn_set_scan_order", int(order))


class Centroids:
    """The IVF centroids on the device, quantised for probe selection (ivf.rs:54-69 `Cent`).

    digits: int8 digit planes (st_knn_centroid_digit_bytes bytes), cexp [nlist] int32,
    cnorm [nlist] float64 (squared norms of the quantised centroids).
    """

    def __init__(self, centroids: torch.Tensor, stream=None):
        if centroids.dim() != 2:
            raise ValueError("centroids must be [nlist, d]")
        nlist, d = centroids.shape
        nbytes = int(_lib.lib().st_knn_centroid_digit_bytes(nlist, d))
        if nbytes < 0:
            raise ValueError(f"probe selection is built for d == 256 (got {d})")
        dev = centroids.device
        self.nlist, self.d = nlist, d
        self.digits = torch.empty(nbytes, dtype=torch.int8, device=dev)
        self.cexp = torch.empty(nlist, dtype=torch.int32, device=dev)
        self.cnorm = torch.empty(nlist, dtype=torch.float64, device=dev)
        _lib.call("st_knn_centroids_prep", _dptr(centroids, torch.float32, "centroids"), nlist, d,
                  self.digits.data_ptr(), self.cexp.data_ptr(), self.cnorm.data_ptr(), _stream(stream))

    def probe(self, queries: torch.Tensor, nprobe: int, out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
        """Each query's nprobe nearest cells, nearest first (ties to the lower id): int32 [nq, nprobe]."""
        nq, d = queries.shape
        if d != self.d:
            raise ValueError(f"queries have width {d}, the centroids {self.d}")
        if out is None:
            out = torch.empty((nq, nprobe), dtype=torch.int32, device=queries.device)
        elif out.shape != (nq, nprobe):
            raise ValueError("out must be [nq, nprobe]")
        _lib.call("st_knn_probe", self.digits.data_ptr(), self.cexp.data_ptr(), self.cnorm.data_ptr(), self.nlist,
                  _dptr(queries, torch.float32, "queries"), nq, d, nprobe, _dptr(out, torch.int32, "probes"),
                  _stream(stream))
        return out


def _check_out(out, nq: int, k: int, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """A caller-supplied (idx, dist) pair must hold nq x k results on the queries' device: the kernels write
    exactly that many and trust the sizes."""
    idx, dist = out
    for t, name in ((idx, "idx"), (dist, "dist")):
        if tuple(t.shape) != (nq, k):
            raise ValueError(f"out {name} must be [{nq}, {k}], got {list(t.shape)}")
        if t.device != device:
            raise ValueError(f"out {name} is on {t.device}, the queries on {device}")
    return idx, dist


class KnnStore2bit:
    """A cell-contiguous 2-bit key store on the device.

    codes [N, d/4] uint8, scales [N] float32 (device tensors); cell_start [ncells+1]
    int64 row offsets (host array; a device copy is kept for the scan).
    """

    def __init__(self, codes: torch.Tensor, scales: torch.Tensor, cell_start, d: int = 256):
        if codes.dim() != 2 or codes.shape[1] * 4 != d:
            raise ValueError("codes must be [N, d/4]")
        if scales.shape != (codes.shape[0],):
            raise ValueError("one scale per key")
        cs = np.ascontiguousarray(np.asarray(cell_start, dtype=np.int64))
        if cs.ndim != 1 or cs.size < 2 or cs[0] != 0 or cs[-1] != codes.shape[0] or np.any(np.diff(cs) < 0):
            raise ValueError("cell_start must rise from 0 to the key count")
        self.d = d
        self.codes = codes
        self.scales = scales
        self.cell_start = cs
        self.ncells = cs.size - 1
        self.max_cell = int(np.diff(cs).max())
        self.cell_start_dev = torch.from_numpy(cs).to(codes.device)
        self.centroids: Optional[Centroids] = None

    def set_centroids(self, centroids: torch.Tensor, stream=None) -> None:
        """Attaches the IVF centroids [ncells, d] (cell c's centroid at row c) for search_ivf by nprobe."""
        if centroids.shape != (self.ncells, self.d):
            raise ValueError(f"need one centroid per cell: [{self.ncells}, {self.d}]")
        self.centroids = Centroids(centroids, stream=stream)

    @classmethod
    def from_keys(cls, keys: torch.Tensor, cell_start, stream=None) -> "KnnStore2bit":
        """Quantises device keys [N, d] (already in cell order) into a store."""
        codes, scales = quantize_2bit(keys, stream=stream)
        return cls(codes, scales, cell_start, keys.shape[1])

    def __len__(self) -> int:
        return self.codes.shape[0]

    def search_ivf(self, queries: torch.Tensor, probes, k: int = KMAX,
                   out: Optional[Tuple[torch.Tensor, torch.Tensor]] = None, stream=None):
        """Per query, the k nearest keys of its probed cells: (idx [nq, k] int64, dist [nq, k] float32).

        queries [nq, d] float32 (device); probes either [nq, nprobe] int32 cell ids (device) or an
        int nprobe, in which case each query probes its nprobe nearest cells (set_centroids first),
        as the reference's search_ivf(queries, rows, nprobe) does.
        """
        if isinstance(probes, int):
            if self.centroids is None:
                raise ValueError("search_ivf by nprobe needs set_centroids")
            probes = self.centroids.probe(queries, probes, stream=stream)
        nq, d = queries.shape
        if d != self.d:
            raise ValueError(f"queries have width {d}, the store {self.d}")
        nprobe = probes.shape[1]
        if probes.shape[0] != nq:
            raise ValueError("one probe row per query")
        if out is None:
            idx = torch.empty((nq, k), dtype=torch.int64, device=queries.device)
            dist = torch.empty((nq, k), dtype=torch.float32, device=queries.device)
        else:
            idx, dist = _check_out(out, nq, k, queries.device)
        _lib.call("st_knn_search_ivf_2bit", _dptr(self.codes, torch.uint8, "codes"),
                  _dptr(self.scales, torch.float32, "scales"), self.cell_start_dev.data_ptr(), self.ncells,
                  self.max_cell, _dptr(queries, torch.float32, "queries"), _dptr(probes, torch.int32, "probes"),
                  nq, nprobe, d, k, _dptr(idx, torch.int64, "idx"), _dptr(dist, torch.float32, "dist"),
                  _stream(stream))
        return idx, dist

    def search_masked(self, queries: torch.Tensor, lohi: torch.Tensor, always: int = 0, k: int = KMAX,
                      out: Optional[Tuple[torch.Tensor, torch.Tensor]] = None, stream=None):
        """The k nearest among keys g < always or lo_i <= g < hi_i (knn.rs:295-331 search_tagged / search_tail):
        (idx [nq, k] int64, dist [nq, k] float32).  lohi [nq, 2] int64 (device), one (lo, hi) range per query."""
        nq, d = queries.shape
        if d != self.d:
            raise ValueError(f"queries have width {d}, the store {self.d}")
        if lohi.shape != (nq, 2):
            raise ValueError("one (lo, hi) range per query")
        if out is None:
            idx = torch.empty((nq, k), dtype=torch.int64, device=queries.device)
            dist = torch.empty((nq, k), dtype=torch.float32, device=queries.device)
        else:
            idx, dist = _check_out(out, nq, k, queries.device)
        _lib.call("st_knn_search_masked_2bit", _dptr(self.codes, torch.uint8, "codes"),
                  _dptr(self.scales, torch.float32, "scales"), len(self), _dptr(queries, torch.float32, "queries"),
                  _dptr(lohi, torch.int64, "lohi"), always, nq, d, k, _dptr(idx, torch.int64, "idx"),
                  _dptr(dist, torch.float32, "dist"), _stream(stream))
        return idx, dist
