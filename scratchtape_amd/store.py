"""The 2-bit store on disk, in the reference's `KnnStore` cache format (gpu_step/knn/cache.rs).

A store built on the device (`knn.quantize_2bit` or `synth_store_2bit`, cells in
order) is written as the reference's `KnnStore::save` writes a quantised store
(cache.rs:33-75), and a file in that format is read back into a device store
(cache.rs:77-135): the reference and this package can exchange stores.

Layout (every integer a little-endian u64; a blob is its byte length then its bytes):
    MAGIC 0x5343_5254_4b4e_4e02, key (blob), extra, d, tile, f16 (1), kbits (2), ntiles,
    per tile: len, codes (rows padded to a multiple of 16, d/4 bytes each, code i at
        byte i/4 bits 2(i%4) as knn.rs:211-214), scales (f32, padded like the rows),
        norms (f32 [len], knn.rs:216), values (f32 [len]),
    the key sample (an empty blob, as the reference now writes it),
    IVF flag; if 1: nlist, n (clustered rows), the centroids as f16 rows padded to a
        multiple of 16 (ivf.rs:433-434), their squared norms (f32 [nlist], ivf.rs:65),
        and per cell its pieces (count, then tile, a, b, g0 each: rows a..b of tile
        `tile` are store rows g0.., ivf.rs:451-462).
"""
from __future__ import annotations

import os
import struct
from typing import BinaryIO, Optional, Tuple

import numpy as np
import torch

from . import _lib
from .knn import KnnStore2bit, _dptr
from .matmul import _stream

MAGIC = 0x5343_5254_4B4E_4E02  # cache.rs:9
KBITS = 2


def _put(w: BinaryIO, x: int) -> None:
    w.write(struct.pack("<Q", x))


def _put_bytes(w: BinaryIO, b) -> None:
    mv = memoryview(b).cast("B")
    _put(w, mv.nbytes)
    w.write(mv)


def _get(r: BinaryIO) -> int:
    b = r.read(8)
    if len(b) != 8:
        raise EOFError("truncated store file")
    return struct.unpack("<Q", b)[0]


def _get_bytes(r: BinaryIO) -> bytes:
    n = _get(r)
    b = r.read(n)
    if len(b) != n:
        raise EOFError("truncated store file")
    return b


def key_norms(codes: torch.Tensor, scales: torch.Tensor, stream=None) -> torch.Tensor:
    """The reference's per-key norms of a quantised store (knn.rs:216), on the device."""
    n, kb = codes.shape
    out = torch.empty(n, dtype=torch.float32, device=codes.device)
    _lib.call("st_knn_key_norms_2bit", _dptr(codes, torch.uint8, "codes"), _dptr(scales, torch.float32, "scales"), n,
              kb * 4, out.data_ptr(), _stream(stream))
    return out


def _f16_rows(x: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Rows rounded to f16 (RNE), padded to a multiple of 16 rows, and their squared norms summed in order in f32."""
    h = x.astype(np.float16)
    norms = np.cumsum(h.astype(np.float32) ** 2, axis=1, dtype=np.float32)[:, -1] if x.shape[1] else \
        np.zeros(x.shape[0], np.float32)
    pad = -x.shape[0] % 16
    return np.concatenate([h, np.zeros((pad, x.shape[1]), np.float16)]), norms.astype(np.float32)


def save(path: str, store: KnnStore2bit, key: str, extra: int = 0, tile: int = 1 << 20,
         values: Optional[np.ndarray] = None, centroids=None) -> None:
    """Writes `store` as the reference's KnnStore::save writes a 2-bit store (through a temporary file).

    values: the keys' byte values (+ DOC) [N] (zeros if None); centroids [ncells, d] (host or device f32) adds the
    IVF section, one cell per store cell (cell_start), as `build_ivf` leaves it.
    """
    n, d = len(store), store.d
    kb = d // 4
    if tile < 16 or tile % 16:
        raise ValueError("tile must be a positive multiple of 16")
    vals = np.zeros(n, np.float32) if values is None else np.asarray(values).astype(np.float32)
    if vals.shape != (n,):
        raise ValueError("one value per key")
    ntiles = -(-n // tile)
    tmp = os.path.splitext(path)[0] + ".part"
    with open(tmp, "wb") as w:
        _put(w, MAGIC)
        _put_bytes(w, key.encode())
        for x in (extra, d, tile, 1, KBITS, ntiles):
            _put(w, x)
        for t in range(ntiles):
            a, b = t * tile, min(n, (t + 1) * tile)
            rows, rp = b - a, -(-(b - a) // 16) * 16
            codes = np.zeros((rp, kb), np.uint8)
            codes[:rows] = store.codes[a:b].cpu().numpy()
            scales = np.zeros(rp, np.float32)
            scales[:rows] = store.scales[a:b].cpu().numpy()
            norms = key_norms(store.codes[a:b], store.scales[a:b]).cpu().numpy()
            _put(w, rows)
            _put_bytes(w, codes)
            _put_bytes(w, scales)
            _put_bytes(w, norms)
            _put_bytes(w, np.ascontiguousarray(vals[a:b]))
        _put_bytes(w, b"")  # the key sample
        if centroids is None:
            _put(w, 0)
        else:
            cent = centroids.cpu().numpy() if isinstance(centroids, torch.Tensor) else np.asarray(centroids, np.float32)
            if cent.shape != (store.ncells, d):
                raise ValueError(f"need one centroid per cell: [{store.ncells}, {d}]")
            c16, cnorm = _f16_rows(cent.astype(np.float32))
            _put(w, 1)
            _put(w, store.ncells)
            _put(w, n)
            _put_bytes(w, c16)
            _put_bytes(w, cnorm)
            cs = store.cell_start
            for c in range(store.ncells):
                pieces = []
                for t in range(ntiles):
                    lo, hi = max(int(cs[c]), t * tile), min(int(cs[c + 1]), (t + 1) * tile)
                    if lo < hi:
                        pieces.append((t, lo - t * tile, hi - t * tile, lo))
                _put(w, len(pieces))
                for p in pieces:
                    for x in p:
                        _put(w, x)
    os.replace(tmp, path)


class Loaded:
    """A store read back from a file: the device store, and what else the file holds."""

    def __init__(self, store, extra, values, norms, centroids, tile):
        self.store: KnnStore2bit = store
        self.extra: int = extra
        self.values: np.ndarray = values        # f32 [N]
        self.norms: np.ndarray = norms          # f32 [N], as stored
        self.centroids: Optional[np.ndarray] = centroids  # f32 [nlist, d] (f16 values) or None
        self.tile: int = tile


def load(path: str, key: str, device="cuda") -> Optional[Loaded]:
    """The store saved at `path` (reference format), or None if there is no such file or it has another key.

    Cells: the IVF cells when the file has them (each a contiguous run of rows, in order, as build_ivf reorders the
    store; rows past the clustered n form one more cell), else one cell of all rows.
    """
    try:
        r = open(path, "rb")
    except OSError:
        return None
    with r:
        if _get(r) != MAGIC or _get_bytes(r) != key.encode():
            return None
        extra, d, tile, _f16, kbits, ntiles = (_get(r) for _ in range(6))
        if kbits != KBITS:
            raise ValueError(f"this store holds {kbits}-bit keys; the 2-bit store reads kbits = 2 only")
        kb = d // 4
        lens, code_parts, scale_parts, norm_parts, val_parts = [], [], [], [], []
        for _ in range(ntiles):
            ln = _get(r)
            cb, sb, nb, vb = _get_bytes(r), _get_bytes(r), _get_bytes(r), _get_bytes(r)
            if len(cb) < ln * kb or len(sb) < ln * 4 or len(nb) != ln * 4 or len(vb) != ln * 4:
                raise ValueError("tile blobs do not match the tile length")
            lens.append(ln)
            code_parts.append(np.frombuffer(cb, np.uint8)[:ln * kb].reshape(ln, kb))
            scale_parts.append(np.frombuffer(sb, np.float32)[:ln])
            norm_parts.append(np.frombuffer(nb, np.float32))
            val_parts.append(np.frombuffer(vb, np.float32))
        r.seek(_get(r), os.SEEK_CUR)  # the key sample
        n = int(sum(lens))
        starts = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        centroids = None
        cell_start = np.array([0, n], np.int64)
        if _get(r) == 1:
            nlist, ncl = _get(r), _get(r)
            cent = np.frombuffer(_get_bytes(r), np.float16)
            _get_bytes(r)  # the centroids' norms (recomputed from the centroids where needed)
            centroids = cent[:nlist * d].reshape(nlist, d).astype(np.float32)
            bounds = [0]
            for c in range(nlist):
                row = bounds[-1]
                for _ in range(_get(r)):
                    t, a, b, g0 = (_get(r) for _ in range(4))
                    if g0 != row or g0 != starts[t] + a or b < a:
                        raise ValueError("IVF cells are not contiguous runs of rows in order")
                    row = g0 + (b - a)
                bounds.append(row)
            if bounds[-1] != ncl:
                raise ValueError("IVF cells do not cover the clustered rows")
            cell_start = np.array(bounds + ([n] if ncl < n else []), np.int64)
    codes = torch.from_numpy(np.concatenate(code_parts) if code_parts else np.zeros((0, kb), np.uint8)).to(device)
    scales = torch.from_numpy(np.concatenate(scale_parts) if scale_parts else np.zeros(0, np.float32)).to(device)
    store = KnnStore2bit(codes, scales, cell_start, d)
    if centroids is not None and store.ncells == centroids.shape[0]:
        store.set_centroids(torch.from_numpy(centroids).to(device))
    return Loaded(store, extra, np.concatenate(val_parts) if val_parts else np.zeros(0, np.float32),
                  np.concatenate(norm_parts) if norm_parts else np.zeros(0, np.float32), centroids, tile)
