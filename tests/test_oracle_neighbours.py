"""Pins the oracle's elementwise neighbours of the matmuls (orc_rmsnorm_residual:
ref:src/kernels/elementwise.cu:463-504; orc_silu_mul: :93-99 then :300-305)
against fp64 numpy and closed forms."""
import numpy as np
import pytest

from conftest import normwise_rel_err


def f64_rmsnorm(x, res, w, eps):
    v = x.astype(np.float64) + (0 if res is None else res.astype(np.float64))
    f = 1.0 / np.sqrt((v * v).mean(axis=1, keepdims=True) + eps)
    return v, v * w.astype(np.float64) * f


@pytest.mark.parametrize("rows,n", [(1, 2048), (16, 2048), (3, 77), (2, 8192)])
def test_rmsnorm_f64(orc, rows, n):
    rng = np.random.default_rng(rows * n)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    r = rng.standard_normal((rows, n)).astype(np.float32) * 0.5
    w = rng.standard_normal(n).astype(np.float32)
    out, normed = orc.rmsnorm_residual(x, r, w, 1e-5)
    v, ref = f64_rmsnorm(x, r, w, 1e-5)
    assert np.array_equal(out, (x + r))           # the residual sum is one fp32 add
    assert normwise_rel_err(normed, ref) < 1e-6


def test_rmsnorm_constant_row_closed_form(orc):
    n, c, eps = 512, 0.75, 1e-5
    x = np.full((1, n), c, np.float32)
    w = np.ones(n, np.float32)
    _, normed = orc.rmsnorm_residual(x, None, w, eps)
    np.testing.assert_allclose(normed, c / np.sqrt(c * c + eps), rtol=2e-7)


def test_rmsnorm_scale_invariance_and_null_residual(orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 300)).astype(np.float32)
    w = rng.standard_normal(300).astype(np.float32)
    _, a = orc.rmsnorm_residual(x, None, w, 0.0)
    _, b = orc.rmsnorm_residual(x * 8.0, None, w, 0.0)       # a power of two: every step exact-scaled
    assert np.array_equal(a, b)
    _, c = orc.rmsnorm_residual(x, np.zeros_like(x), w, 0.0)
    assert np.array_equal(a, c)


def test_silu_mul(orc):
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(10000) * 4).astype(np.float32)
    u = rng.standard_normal(10000).astype(np.float32)
    out = orc.silu_mul(g, u)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert normwise_rel_err(out, ref) < 1e-6
    ends = orc.silu_mul(np.array([0.0, 60.0, -60.0, -0.0], np.float32), np.ones(4, np.float32))
    assert ends[0] == 0.0 and ends[1] == 60.0 and abs(ends[2]) < 1e-20 and ends[3] == 0.0
