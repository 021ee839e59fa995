"""CPU checks of the boundary: the library loads, exports every symbol the header
declares, and the host-side mirrors validate arguments as the reference asserts."""
import os
import re

import numpy as np
import pytest

import scratchtape_amd
from scratchtape_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "scratchtape_hip.h")


def header_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(st_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    syms = header_symbols()
    for name in ["st_matmul", "st_matmul_f32", "st_matmul_with", "st_ndarray_matmul", "st_softmax",
                 "st_softmax_backward", "st_knn_quantize_2bit", "st_knn_search_ivf_2bit", "st_last_error"]:
        assert name in syms


def test_library_exports_every_declared_symbol():
    L = scratchtape_amd.lib()
    for name in header_symbols():
        assert hasattr(L, name), name
    # and the Python binding covers them all with argtypes
    assert set(header_symbols()) == set(_lib.SIGNATURES)


def test_version_and_f16_switch():
    L = scratchtape_amd.lib()
    assert L.st_version().startswith(b"scratchtape_hip")
    assert L.st_f16_enabled() in (0, 1)


def test_struct_layouts_match_the_header():
    # st_matref: p, off, stride, trans, reserved, ld, group, inner
    assert _lib.StMatRef.inner.offset == 48 and _lib.ctypes.sizeof(_lib.StMatRef) == 56
    assert _lib.StEpilogue.col_sum_stride.offset == 80 and _lib.ctypes.sizeof(_lib.StEpilogue) == 88
    # st_gemm: a, b, out (st_matref), epi, batch, m, k, n, use_f16, reserved
    assert _lib.StGemm.epi.offset == 168 and _lib.StGemm.batch.offset == 256
    assert _lib.StGemm.use_f16.offset == 288 and _lib.ctypes.sizeof(_lib.StGemm) == 296


def test_null_arguments_are_rejected_without_a_device():
    L = scratchtape_amd.lib()
    rc = L.st_matmul(None, None, None, 1, 1, 1, 1, None, None)
    assert rc == _lib.ST_ERR_INVALID
    assert b"NULL" in L.st_last_error()
    rc = L.st_softmax(None, None, 4, 4, 4, 1.0, 1, 0, None)
    assert rc == _lib.ST_ERR_INVALID
    rc = L.st_matmul_grouped(None, 2, None)
    assert rc == _lib.ST_ERR_INVALID
    g = (_lib.StGemm * 2)()
    g[1].batch, g[1].m, g[1].k, g[1].n = 1, 4, 4, 4   # g[1].a.p is NULL
    rc = L.st_matmul_grouped(g, 2, None)
    assert rc == _lib.ST_ERR_INVALID and b"GEMM 0 of the group" in L.st_last_error()


def test_ndarray_matmul_shape_asserts_like_the_reference():
    from scratchtape_amd.tensor import ndarray_matmul
    with pytest.raises(ValueError, match="inner dims must match"):
        ndarray_matmul(np.zeros((2, 3), np.float32), np.zeros((4, 2), np.float32))
    with pytest.raises(ValueError, match="lhs must be 2D"):
        ndarray_matmul(np.zeros(3, np.float32), np.zeros((3, 2), np.float32))


def test_f16_route_mirrors_the_reference_pick():
    from scratchtape_amd import f16_route
    assert f16_route(128, 64, 64) and f16_route(128, 64, 96)
    assert not f16_route(70, 64, 64)          # m ragged
    assert not f16_route(64, 48, 64)          # k not a multiple of 32
    assert not f16_route(64, 64, 64, col_sum=True, b_trans=True)
    assert f16_route(4096, 256, 768)


def test_probe_arguments_are_validated_like_the_reference_asserts():
    # ivf.rs:469 asserts nprobe in 1..=min(nlist, PROBE_MAX); the width is the scan's 256.
    L = scratchtape_amd.lib()
    fake = 1 << 20  # aligned non-null stand-in: every call below is rejected before any access
    assert L.st_knn_centroid_digit_bytes(12288, 256) == 1536 * 4096
    assert L.st_knn_centroid_digit_bytes(9, 256) == 2 * 4096
    assert L.st_knn_centroid_digit_bytes(9, 128) == -1
    cases = [
        ((None, fake, fake, 64, fake, 4, 256, 8, fake, None), b"NULL"),
        ((fake, fake, fake, 64, fake, 4, 128, 8, fake, None), b"d == 256"),
        ((fake, fake, fake, 64, fake, 4, 256, 17, fake, None), b"nprobe"),
        ((fake, fake, fake, 64, fake, 4, 256, 0, fake, None), b"nprobe"),
        ((fake, fake, fake, 4, fake, 4, 256, 5, fake, None), b"nprobe"),
        ((fake, fake, fake, 64, fake + 4, 4, 256, 8, fake, None), b"aligned"),
    ]
    for args, msg in cases:
        assert L.st_knn_probe(*args) == _lib.ST_ERR_INVALID
        assert msg in L.st_last_error(), (args, L.st_last_error())
    assert L.st_knn_centroids_prep(fake, 64, 200, fake, fake, fake, None) == _lib.ST_ERR_INVALID
    assert L.st_knn_centroids_prep(fake, 0, 256, fake, fake, fake, None) == _lib.ST_ERR_INVALID


def test_fused_attention_arguments_are_validated():
    L = scratchtape_amd.lib()
    fake = 1 << 20
    for (b, h, t, hd), msg in [((32, 4, 128, 32), b"head_dim 64"), ((32, 4, 100, 64), b"multiple of 32"),
                               ((32, 4, 288, 64), b"multiple of 32"), ((0, 4, 128, 64), b"batch")]:
        assert L.st_attention_fused_fwd(fake, fake, fake, b, h, t, hd, 0.125, 0, None) == _lib.ST_ERR_INVALID
        assert msg in L.st_last_error()
        assert L.st_attention_fused_bwd(fake, fake, fake, fake, fake, b, h, t, hd, 0.125, None) == _lib.ST_ERR_INVALID
    assert L.st_attention_fused_fwd(None, fake, fake, 32, 4, 128, 64, 0.125, 0, None) == _lib.ST_ERR_INVALID


def test_layer_norm_arguments_are_validated():
    L = scratchtape_amd.lib()
    fake = 1 << 20
    assert L.st_layer_norm(None, 4, 8, fake, 0, 1e-5, 1, 0, fake, fake, fake, None) == _lib.ST_ERR_INVALID
    assert L.st_layer_norm(fake, 5, 8, fake, 0, 1e-5, 2, 16, fake, fake, fake, None) == _lib.ST_ERR_INVALID
    assert b"split evenly" in L.st_last_error()
    assert L.st_layer_norm_backward(fake, fake, fake, fake, 4, 8, fake, fake, 0, fake, 0, 2, 8, None) == \
        _lib.ST_ERR_INVALID
    assert b"overlap" in L.st_last_error()


def test_masked_search_arguments_are_validated():
    L = scratchtape_amd.lib()
    fake = 1 << 20
    assert L.st_knn_search_masked_2bit(fake, fake, 100, fake, fake, 0, 4, 256, 128, fake, fake, None) == \
        _lib.ST_ERR_INVALID
    assert b"at least 128 keys" in L.st_last_error()
    assert L.st_knn_search_masked_2bit(fake, fake, 1000, fake, fake, 0, 4, 128, 128, fake, fake, None) == \
        _lib.ST_ERR_INVALID
    assert L.st_knn_search_masked_2bit(fake, fake, 1000, fake, fake, 0, 4, 256, 129, fake, fake, None) == \
        _lib.ST_ERR_INVALID


def test_ceiling_probe_arguments_are_validated():
    L = scratchtape_amd.lib()
    fake = 1 << 20
    assert L.st_peak_mfma(5, 10, 8, fake, None) == _lib.ST_ERR_INVALID
    assert b"kind" in L.st_last_error()
    assert L.st_peak_mfma(0, 0, 8, fake, None) == _lib.ST_ERR_INVALID
    assert L.st_peak_read(fake, 24, 8, fake, None) == _lib.ST_ERR_INVALID
    assert L.st_peak_read(fake + 4, 32, 8, fake, None) == _lib.ST_ERR_INVALID
    assert L.st_lane_selftest(None, None) == _lib.ST_ERR_INVALID
    assert L.st_device_info(None, None, None, None) == _lib.ST_ERR_INVALID


def test_caller_outputs_are_size_checked_before_any_device_call():
    """A caller-supplied out smaller than what the kernel writes is refused on the host (CPU tensors: the
    check runs before the C ABI is reached)."""
    import torch

    from scratchtape_amd import rows
    from scratchtape_amd.knn import KnnStore2bit

    store = KnnStore2bit(torch.zeros((300, 64), dtype=torch.uint8), torch.ones(300), [0, 100, 300])
    q = torch.zeros((3, 256))
    probes = torch.zeros((3, 2), dtype=torch.int32)
    good = (torch.empty((3, 128), dtype=torch.int64), torch.empty((3, 128)))
    for bad in ((torch.empty((3, 127), dtype=torch.int64), good[1]), (good[0], torch.empty((2, 128))),
                (good[0], torch.empty(3 * 128))):
        with pytest.raises(ValueError, match="out"):
            store.search_ivf(q, probes, out=bad)
        with pytest.raises(ValueError, match="out"):
            store.search_masked(q, torch.zeros((3, 2), dtype=torch.int64), out=bad)
    x = torch.zeros(4 * 8)
    with pytest.raises(ValueError, match="writes 32"):
        rows.softmax(x, 4, 8, 8, 1.0, True, False, out=torch.empty(31))
    with pytest.raises(ValueError, match="writes 32"):
        rows.softmax_backward(x, x, 4, 8, 1.0, out=torch.empty(16))


def test_scratch_release_without_arenas_is_a_no_op():
    L = scratchtape_amd.lib()
    if L.st_scratch_release() != _lib.ST_OK:
        # No HIP device in this process: the call reports it instead of crashing.
        assert L.st_last_error()
