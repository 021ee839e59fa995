"""CPU oracle for the scratchtape matrix-multiplication hot path.

TEST INFRASTRUCTURE ONLY: what ``tests/`` and the package ``__graft_entry__.smoke()``
compare the library against, and ``bench.py``'s CPU baseline.  The product
library (``scratchtape_amd``) never imports this module.

The arithmetic lives in ``oracle.c`` (built to ``liboracle.so`` by the Makefile
beside it); this module only wraps it with numpy.  Each function names the
reference code it restates and how it is pinned (the test that pins it):

=====================  =========================================  ======================================================
function               reference                                  pinned by (tests/test_oracle.py)
=====================  =========================================  ======================================================
Rng                    src/nn.rs:8-35 (xorshift64 13/7/17)        Marsaglia's published xorshift64 outputs; big-int
                                                                   recurrence; next_f32 range; Box-Muller moments
matmul                 src/tensor.rs:241-276                      gpu.rs:176-185 KAT; integer-valued inputs vs exact
                                                                   int64 products; identity/permutation; float64 bound;
                                                                   bit-equality with an independent p-ascending
                                                                   float32 accumulation and inequality with FMA order
transpose              src/tensor.rs:278-287                      involution, numpy .T
round_f16              half 2.7.1 from_f32 (RNE)                  IEEE-754 tie/overflow/subnormal KATs; numpy float16
gemm (MatRef/Epilogue)  gpu_step/matmul.rs:26-79, 888-937         integer-valued exactness vs numpy int64 per epilogue
                                                                   term; head views vs explicit split_heads slicing
layer_norm / backward  nn.rs:306-321, gpu_step/rows.rs:60-99,     float64 closed form; mean 0 / variance 1 of the
                       177-293                                    normalised rows; finite-difference dx; dgamma/dbeta
                                                                   as column sums; per-model parameter sets
softmax / backward     gpu_step/rows.rs:101-123, 295-357          float64 softmax; rows sum to 1; masked entries exactly
                                                                   0; finite-difference gradient; softmax1 phantom term
attention_fwd_bwd      src/tape.rs:73-112 (+ causal mask)         float64 closed-form attention forward and gradients
quantize_2bit          gpu_step/knn.rs:190-225 (bits 2)           hand-computed rows (ties round away from zero, clamp,
                                                                   packing order, 1e-30 floor); float64 scale formula
knn_prep_query         build contract (int16 query)               exactness: Q*qs reproduces q to half an ulp of qs;
                                                                   power-of-two qs; |Q| range
knn_search             build contract (ivf.rs:235 distance,       int64 brute force + numpy float32 formula + lexsort;
                       ivf.rs:673-684 finalisation)               exact integer dot vs float64; fidelity to the
                                                                   reference's own f16 scoring within its 2e-3 tolerance
knn_search_masked      knn.rs:295-331 search_tagged/search_tail,  the IVF brute force with the mask predicate; equality
                       key predicate knn.rs:604-618               with knn_search when the range is one cell; always
                                                                   prefix, empty and clipped ranges
knn_centroid_prep      ivf.rs:62-69 Cent::new, with the scan's     exactness: C * 2^cexp reproduces the centroid as
                       int16 quantiser in place of f16 rounding  knn_prep_query does; cnorm = float64 |C 2^cexp|^2
knn_probe              ivf.rs:128-161 k_probe over the dots of     float64 brute force of |q - c|^2 (ranking agrees
                       ivf.rs:473-484                             wherever the gap exceeds the quantisation bound); a
                                                                   query equal to a centroid probes it first; duplicate
                                                                   centroids tie to the lower id; permutation covariance;
                                                                   nprobe = nlist is a full sort
=====================  =========================================  ======================================================
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_i16p = np.ctypeslib.ndpointer(dtype=np.int16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_u64 = ctypes.c_uint64
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32


class _MatRef(ctypes.Structure):
    _fields_ = [("off", _i64), ("stride", _i64), ("trans", _i64), ("ld", _i64), ("group", _i64), ("inner", _i64)]


class QPrep(ctypes.Structure):
    _fields_ = [("qs", ctypes.c_float), ("qn", ctypes.c_float), ("sq", _i32), ("qe", _i32)]


def build() -> None:
    """Compile liboracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_rng_next_f32.argtypes = [ctypes.POINTER(_u64)]
        L.orc_rng_next_f32.restype = ctypes.c_float
        L.orc_rng_next_gaussian.argtypes = [ctypes.POINTER(_u64)]
        L.orc_rng_next_gaussian.restype = ctypes.c_float
        L.orc_rng_fill_uniform.argtypes = [ctypes.POINTER(_u64), _i64, _f32p]
        L.orc_rng_fill_gaussian.argtypes = [ctypes.POINTER(_u64), _i64, ctypes.c_float, _f32p]
        L.orc_matmul.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64]
        L.orc_transpose.argtypes = [_f32p, _f32p, _i64, _i64]
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_round_f16_array.argtypes = [_f32p, _f32p, _i64]
        L.orc_gemm.argtypes = [
            _f32p, ctypes.POINTER(_MatRef), _f32p, ctypes.POINTER(_MatRef), _f32p, ctypes.POINTER(_MatRef),
            _i64, _i64, _i64, _i64,
            ctypes.c_void_p, _i64, _i32, ctypes.c_void_p, ctypes.c_void_p, _i32, _i32, _i64, _i64, _i32,
        ]
        L.orc_softmax.argtypes = [_f32p, _f32p, _i64, _i64, _i64, ctypes.c_float, _i32, _i32]
        L.orc_softmax_backward.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, ctypes.c_float]
        L.orc_attention_fwd_bwd.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, ctypes.c_float, _i32,
                                            _f32p, _f32p, _f32p, _f32p, _f32p, _f32p]
        L.orc_quantize_2bit.argtypes = [_f32p, _i64, _i64, _u8p, _f32p, ctypes.c_void_p]
        L.orc_knn_prep_query.argtypes = [_f32p, _i64, _i16p, ctypes.POINTER(QPrep)]
        L.orc_knn_dists.argtypes = [_u8p, _f32p, _i64, _i64, _i64, _i16p, ctypes.POINTER(QPrep), _f32p]
        L.orc_knn_search.argtypes = [_u8p, _f32p, _i64p, _f32p, _i32p, _i64, _i64, _i64, _i64, _i64p, _f32p]
        L.orc_knn_search_masked.argtypes = [_u8p, _f32p, _i64, _f32p, _i64p, _i64p, _i64, _i64, _i64, _i64, _i64p,
                                             _f32p]
        L.orc_knn_ref_f16_dist.argtypes = [_u8p, ctypes.c_float, ctypes.c_float, _f32p, _i64]
        L.orc_knn_ref_f16_dists.argtypes = [_u8p, _f32p, _f32p, _i64, _i64, _i64, _f32p, _f32p]
        L.orc_knn_ref_f16_probe.argtypes = [_f32p, _i64, _f32p, _i64, _i64, _i64, _i32p]
        L.orc_layer_norm.argtypes = [_f32p, _i64, _i64, _f32p, _i64, ctypes.c_float, _i64, _i64, _f32p, _f32p, _f32p]
        L.orc_layer_norm_backward.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _f32p, _f32p, _i64, _f32p, _i32,
                                              _i64, _i64]
        L.orc_knn_centroid_prep.argtypes = [_f32p, _i64, _i64, _i16p, _i32p, _f64p]
        L.orc_knn_probe.argtypes = [_i16p, _i32p, _f64p, _i64, _f32p, _i64, _i64, _i64, _i32p]
        L.orc_knn_ref_f16_dist.restype = ctypes.c_float
        L.orc_set_threads.argtypes = [_i32]
        L.orc_get_threads.restype = _i32
        _lib = L
    return _lib


class threads:
    """Context manager: matmul, transpose and knn_search split their rows (queries) over n OpenMP threads inside
    the block (1 outside, the reference's single-threaded path).  Results are the same for every n; only the
    all-cores CPU baseline uses more than one."""

    def __init__(self, n: int):
        self.n = max(1, int(n))

    def __enter__(self):
        self.old = lib().orc_get_threads()
        lib().orc_set_threads(self.n)
        return self

    def __exit__(self, *exc):
        lib().orc_set_threads(self.old)


# --------------------------------------------------------------------------- Rng (nn.rs:8-35)

class Rng:
    """xorshift64 state with the reference's next_f32 / next_gaussian."""

    def __init__(self, seed: int):
        self.state = _u64(seed)

    def next_f32(self) -> float:
        return lib().orc_rng_next_f32(ctypes.byref(self.state))

    def next_gaussian(self) -> float:
        return lib().orc_rng_next_gaussian(ctypes.byref(self.state))

    def uniform(self, n: int) -> np.ndarray:
        """n values of next_f32()*2-1 (gpu.rs:189-192)."""
        out = np.empty(n, np.float32)
        lib().orc_rng_fill_uniform(ctypes.byref(self.state), n, out)
        return out

    def gaussian(self, n: int, scale: float = 1.0) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib().orc_rng_fill_gaussian(ctypes.byref(self.state), n, scale, out)
        return out


# --------------------------------------------------------------------------- tensor.rs

def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """NdArray::matmul (tensor.rs:241-276), bit-exact restatement."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    assert a.ndim == 2 and b.ndim == 2, "matmul is 2D only"
    m, k = a.shape
    k2, n = b.shape
    assert k == k2, f"matmul inner dims must match: {a.shape} vs {b.shape}"
    out = np.empty((m, n), np.float32)
    lib().orc_matmul(a, b, out, m, k, n)
    return out


def transpose(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    m, n = a.shape
    out = np.empty((n, m), np.float32)
    lib().orc_transpose(a, out, m, n)
    return out


def round_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().orc_round_f16_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def f32_to_f16_bits(x: float) -> int:
    return int(lib().orc_f32_to_f16(float(x)))


# --------------------------------------------------------------------------- gpu_step::matmul semantics

def _ref(off=0, stride=0, trans=False, ld=0, group=1, inner=0) -> _MatRef:
    return _MatRef(off, stride, int(bool(trans)), ld, group, inner)


def gemm(a_buf, a, b_buf, b, out_buf, out, batch, m, k, n, *, bias=None, bias_stride=0, relu=False,
         mask=None, residual=None, accumulate=False, col_sum=None, f16=False):
    """gpu_step::matmul's meaning (matmul.rs:62-106) on host buffers, in place on out_buf.

    a, b, out are dicts with MatRef fields (off, stride, trans, ld, group, inner);
    bias/mask/residual are (buffer, offset) pairs; col_sum is (offset, stride) into out_buf.
    """
    a_buf = np.ascontiguousarray(a_buf, np.float32)
    b_buf = np.ascontiguousarray(b_buf, np.float32)
    assert out_buf.dtype == np.float32 and out_buf.flags.c_contiguous
    keep = []

    def ptr(pair):
        if pair is None:
            return None
        buf, off = pair
        buf = np.ascontiguousarray(buf, np.float32)
        keep.append(buf)
        return buf.ctypes.data + 4 * off

    cs_off, cs_stride = col_sum if col_sum is not None else (0, 0)
    lib().orc_gemm(a_buf, ctypes.byref(_ref(**a)), b_buf, ctypes.byref(_ref(**b)), out_buf,
                   ctypes.byref(_ref(**out)), batch, m, k, n, ptr(bias), bias_stride, int(relu),
                   ptr(mask), ptr(residual), int(accumulate), int(col_sum is not None), cs_off, cs_stride,
                   int(f16))
    return out_buf


# --------------------------------------------------------------------------- rows.rs

def softmax(x: np.ndarray, rows: int, n: int, t: int, scale: float, causal: bool, one: bool) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    y = np.empty(rows * n, np.float32)
    lib().orc_softmax(x, y, rows, n, t, scale, int(causal), int(one))
    return y


def softmax_backward(dy: np.ndarray, y: np.ndarray, rows: int, n: int, scale: float) -> np.ndarray:
    dy = np.ascontiguousarray(dy, np.float32).reshape(-1)
    y = np.ascontiguousarray(y, np.float32).reshape(-1)
    dx = np.empty(rows * n, np.float32)
    lib().orc_softmax_backward(dy, y, dx, rows, n, scale)
    return dx


def attention_fwd_bwd(q, k, v, dout, chunks, t, hd, scale, one=False):
    """Per-chunk CPU attention forward + backward (tape.rs:73-112): returns P, O, dQ, dK, dV (one: softmax1)."""
    arrs = [np.ascontiguousarray(x, np.float32).reshape(-1) for x in (q, k, v, dout)]
    p = np.empty(chunks * t * t, np.float32)
    o, dq, dk, dv = (np.empty(chunks * t * hd, np.float32) for _ in range(4))
    scratch = np.empty(4 * t * t + 3 * t * hd, np.float32)
    lib().orc_attention_fwd_bwd(*arrs, chunks, t, hd, scale, int(one), p, o, dq, dk, dv, scratch)
    return p, o, dq, dk, dv


def layer_norm(x, rows, d, params, off, eps=1e-5, rows_pm=None, stride=0):
    """LayerNorm forward (nn.rs:306-321): returns (y, mean, rstd); rows_pm rows per parameter set."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    params = np.ascontiguousarray(params, np.float32)
    y = np.empty(rows * d, np.float32)
    mean, rstd = np.empty(rows, np.float32), np.empty(rows, np.float32)
    lib().orc_layer_norm(x, rows, d, params, off, eps, rows_pm or rows, stride, y, mean, rstd)
    return y, mean, rstd


def layer_norm_backward(dy, x, mean, rstd, rows, d, params, grads, off, dx=None, accumulate=False, rows_pm=None,
                        stride=0):
    """LayerNorm backward: returns dx; adds the gamma/beta gradients into grads (a float32 array, in place)."""
    dy = np.ascontiguousarray(dy, np.float32).reshape(-1)
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    dx = np.zeros(rows * d, np.float32) if dx is None else np.ascontiguousarray(dx, np.float32).copy()
    assert grads.dtype == np.float32 and grads.flags.c_contiguous
    lib().orc_layer_norm_backward(dy, x, np.ascontiguousarray(mean, np.float32), np.ascontiguousarray(rstd, np.float32),
                                  rows, d, np.ascontiguousarray(params, np.float32), grads, off, dx, int(accumulate),
                                  rows_pm or rows, stride)
    return dx


# --------------------------------------------------------------------------- kNN (knn.rs, ivf.rs)

def quantize_2bit(keys: np.ndarray, d: int, with_norm: bool = False):
    """tile_of for 2-bit keys (knn.rs:190-225): codes [n, d/4] u8, scales [n] f32 (+ the f16 norms)."""
    keys = np.ascontiguousarray(keys, np.float32).reshape(-1)
    n = keys.size // d
    codes = np.empty((n, d // 4), np.uint8)
    scales = np.empty(n, np.float32)
    norm = np.empty(n, np.float32) if with_norm else None
    lib().orc_quantize_2bit(keys, n, d, codes, scales, norm.ctypes.data if with_norm else None)
    return (codes, scales, norm) if with_norm else (codes, scales)


def knn_prep_query(q: np.ndarray):
    q = np.ascontiguousarray(q, np.float32).reshape(-1)
    Q = np.empty(q.size, np.int16)
    prep = QPrep()
    lib().orc_knn_prep_query(q, q.size, Q, ctypes.byref(prep))
    return Q, prep


def knn_dists(codes, scales, d, r0, r1, q):
    Q, prep = knn_prep_query(q)
    out = np.empty(r1 - r0, np.float32)
    lib().orc_knn_dists(np.ascontiguousarray(codes).reshape(-1), np.ascontiguousarray(scales), d, r0, r1, Q,
                        ctypes.byref(prep), out)
    return out


def knn_search(codes, scales, cell_start, queries, probes, k=128):
    """Top-k by (dist, key index) over each query's probed cells; returns (idx int64 [nq,k], dist f32 [nq,k])."""
    codes = np.ascontiguousarray(codes, np.uint8).reshape(-1)
    scales = np.ascontiguousarray(scales, np.float32)
    cell_start = np.ascontiguousarray(cell_start, np.int64)
    probes = np.ascontiguousarray(probes, np.int32)
    nq, nprobe = probes.shape
    d = (codes.size // scales.size) * 4
    queries = np.ascontiguousarray(queries, np.float32).reshape(nq, d)
    idx = np.empty((nq, k), np.int64)
    dist = np.empty((nq, k), np.float32)
    lib().orc_knn_search(codes, scales, cell_start, queries.reshape(-1), probes, nq, nprobe, d, k, idx, dist)
    return idx, dist


def knn_search_masked(codes, scales, queries, lo, hi, always=0, k=128):
    """Top-k by (dist, key index) over keys g < always or lo[i] <= g < hi[i] (knn.rs:295-331, 604-618)."""
    codes = np.ascontiguousarray(codes, np.uint8).reshape(-1)
    scales = np.ascontiguousarray(scales, np.float32)
    queries = np.ascontiguousarray(queries, np.float32)
    nq, d = queries.shape
    idx = np.empty((nq, k), np.int64)
    dist = np.empty((nq, k), np.float32)
    lib().orc_knn_search_masked(codes, scales, scales.size, queries.reshape(-1), np.ascontiguousarray(lo, np.int64),
                                np.ascontiguousarray(hi, np.int64), always, nq, d, k, idx.reshape(-1), dist.reshape(-1))
    return idx, dist


def knn_ref_f16_dist(code_row, scale, norm_f16, q):
    return lib().orc_knn_ref_f16_dist(np.ascontiguousarray(code_row, np.uint8), float(scale), float(norm_f16),
                                      np.ascontiguousarray(q, np.float32), q.size)


def knn_ref_f16_dists(codes, scales, norm_f16, r0, r1, q):
    """knn_ref_f16_dist for keys r0..r1 of a store against one query: float32 [r1 - r0]."""
    codes = np.ascontiguousarray(codes, np.uint8).reshape(-1)
    scales = np.ascontiguousarray(scales, np.float32)
    d = (codes.size // scales.size) * 4
    out = np.empty(r1 - r0, np.float32)
    lib().orc_knn_ref_f16_dists(codes, scales, np.ascontiguousarray(norm_f16, np.float32), d, r0, r1,
                                np.ascontiguousarray(q, np.float32), out)
    return out


def knn_ref_f16_probe(cent: np.ndarray, queries: np.ndarray, nprobe: int) -> np.ndarray:
    """The reference's f16 probe ranking (ivf.rs:62-67, 470-485, 131-161): int32 [nq, nprobe], nearest first."""
    cent = np.ascontiguousarray(cent, np.float32)
    queries = np.ascontiguousarray(queries, np.float32)
    nq, d = queries.shape
    out = np.empty((nq, nprobe), np.int32)
    lib().orc_knn_ref_f16_probe(cent.reshape(-1), cent.shape[0], queries.reshape(-1), nq, d, nprobe, out.reshape(-1))
    return out


def knn_centroid_prep(cent: np.ndarray):
    """Centroids [nlist, d] f32 -> (C int16 [nlist, d], cexp int32 [nlist], cnorm float64 [nlist])."""
    cent = np.ascontiguousarray(cent, np.float32)
    nlist, d = cent.shape
    C = np.empty((nlist, d), np.int16)
    cexp = np.empty(nlist, np.int32)
    cnorm = np.empty(nlist, np.float64)
    lib().orc_knn_centroid_prep(cent.reshape(-1), nlist, d, C.reshape(-1), cexp, cnorm)
    return C, cexp, cnorm


def knn_probe(cent: np.ndarray, queries: np.ndarray, nprobe: int, prep=None) -> np.ndarray:
    """Each query's nprobe nearest cells by (dd, cell id), nearest first: int32 [nq, nprobe]."""
    C, cexp, cnorm = prep if prep is not None else knn_centroid_prep(cent)
    queries = np.ascontiguousarray(queries, np.float32)
    nq, d = queries.shape
    out = np.empty((nq, nprobe), np.int32)
    lib().orc_knn_probe(np.ascontiguousarray(C).reshape(-1), cexp, cnorm, C.shape[0], queries.reshape(-1), nq, d,
                        nprobe, out.reshape(-1))
    return out
