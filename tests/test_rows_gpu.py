"""LayerNorm forward and backward on the GPU against the CPU oracle (nn.rs:306-321 on
the CPU tape; gpu_step/rows.rs:60-99, 177-293 on the device), as the reference's own
layer_norm_matches_cpu_tape (rows.rs:405-454) checks them: y within 1e-5, dx, dgamma
and dbeta within 1e-4 (scale-relative), gamma/beta at an offset in a flat parameter
buffer with nothing written outside, accumulate doubling dx."""
import random

import numpy as np
import pytest
import torch

import oracle
from scratchtape_amd import rows

pytestmark = pytest.mark.gpu


def rel_err(got, want):
    return float(np.max(np.abs(got - want))) / max(float(np.max(np.abs(want))), 1e-30)


def params_flat(d, off, models=1, stride=None):
    stride = stride if stride is not None else 2 * d
    flat = np.full(off + (models - 1) * stride + 2 * d + 1, 9.0, np.float32)
    j = np.arange(d)
    for m in range(models):
        flat[off + m * stride: off + m * stride + d] = 1.0 + 0.1 * ((j * 7 + m) % 5)
        flat[off + m * stride + d: off + m * stride + 2 * d] = 0.05 * ((j * 3 + m) % 4) - 0.1
    return flat, stride


def run_case(dev, nrows, d, off, models=1, stride=None, seed=7):
    params, stride = params_flat(d, off, models, stride)
    rng = oracle.Rng(seed)
    x, r = rng.gaussian(nrows * d), rng.gaussian(nrows * d)
    rows_pm = nrows // models
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    xh, rh, ph = T(x), T(r), T(params)
    fwd = rows.layer_norm(xh, nrows, d, ph, off, 1e-5, models, stride)
    y, mean, rstd = oracle.layer_norm(x, nrows, d, params, off, 1e-5, rows_pm, stride)
    assert rel_err(fwd.y.cpu().numpy(), y) < 1e-5
    assert rel_err(fwd.mean.cpu().numpy(), mean) < 1e-5 and rel_err(fwd.rstd.cpu().numpy(), rstd) < 1e-5
    grads = T(np.full(params.size, 0.5, np.float32))
    dx = T(np.zeros(nrows * d, np.float32))
    rows.layer_norm_backward(rh, xh, fwd, nrows, d, ph, grads, off, dx, False, models, stride)
    wg = np.full(params.size, 0.5, np.float32)
    wdx = oracle.layer_norm_backward(r, x, mean, rstd, nrows, d, params, wg, off, rows_pm=rows_pm, stride=stride)
    assert rel_err(dx.cpu().numpy(), wdx) < 1e-4
    g = grads.cpu().numpy()
    for m in range(models):
        a = off + m * stride
        assert rel_err(g[a:a + d], wg[a:a + d]) < 1e-4, "dgamma"
        assert rel_err(g[a + d:a + 2 * d], wg[a + d:a + 2 * d]) < 1e-4, "dbeta"
    mask = np.ones(params.size, bool)
    for m in range(models):
        mask[off + m * stride: off + m * stride + 2 * d] = False
    assert np.all(g[mask] == 0.5), "wrote outside gamma/beta"
    rows.layer_norm_backward(rh, xh, fwd, nrows, d, ph, grads, off, dx, True, models, stride)
    assert rel_err(dx.cpu().numpy(), 2 * wdx) < 1e-4, "dx accumulate"


@pytest.mark.parametrize("nrows,d,off", [(37, 24, 5), (37, 200, 3), (203, 24, 5)])
def test_layer_norm_reference_cases(dev, nrows, d, off):
    run_case(dev, nrows, d, off)


def test_layer_norm_at_the_step_shape(dev):
    # T = 4096 tokens of d_model 256: 32 column-sum chunks per column.
    run_case(dev, 4096, 256, 0, seed=11)


def test_layer_norm_two_models_with_strided_parameter_sets(dev):
    run_case(dev, 2 * 300, 100, 4, models=2, stride=3 * 100 + 7, seed=13)


# The vector forms (d % 4 == 0 up to 1024, 16-byte aligned rows and parameter sets): the backward's row pass
# writes dx and per-16-row-chunk column partials, a second launch adds the chunks (one or several per slice).
@pytest.mark.parametrize("nrows,d,off", [(37, 24, 4), (203, 200, 8), (600, 520, 0), (300, 1024, 4), (5, 256, 0)])
def test_layer_norm_vector_forms(dev, nrows, d, off):
    run_case(dev, nrows, d, off, seed=nrows + d)


def test_layer_norm_vector_forms_three_models(dev):
    # 272 rows per model: 17 chunks per model, over sixteen slices of two chunks (the last slice empty).
    run_case(dev, 3 * 272, 64, 8, models=3, stride=2 * 64 + 12, seed=17)


@pytest.mark.parametrize("nrows,d,off", [(64, 1028, 0), (64, 250, 0), (64, 256, 2)])
def test_layer_norm_falls_back_off_the_vector_forms(dev, nrows, d, off):
    run_case(dev, nrows, d, off, seed=3)


def test_layer_norm_back_to_back_shapes(dev):
    """Calls of different shapes back to back, each checked (the row scratch arena is reused across them)."""
    for nrows, d in [(4096, 256), (37, 24), (600, 520), (4096, 256)]:
        run_case(dev, nrows, d, 0, seed=nrows)


def test_layer_norm_random_shapes(dev):
    # Seeded random shapes: widths 1..1100 (vector and scalar forms), parameter offsets 0..8,
    # one to three models, rows 1..700.
    rnd = random.Random(19)
    for i in range(10):
        models = rnd.choice([1, 1, 2, 3])
        nrows = models * rnd.randint(1, 700 // models)
        d = rnd.choice([rnd.randint(1, 1100), 4 * rnd.randint(1, 256)])
        run_case(dev, nrows, d, rnd.randint(0, 8), models, seed=40 + i)
