"""The product-side numpy quantizers (cretif_amd/quant.py, used to make
synthetic weights) are byte-identical to the oracle's scalar restatements of
the reference quantizers (ref:tests/test_matmul_quant.cu) -- two separate
implementations checking each other."""
import numpy as np
import pytest

from cretif_amd import quant

CASES = {
    "q8_0": "q8_0",
    "q4_0": "q4_0",
    "q5_0": "q5_0",
    "q6_k": "q6_k",
    "q4_k": "q4_k_asym",
}


def _inputs(seed, n):
    rng = np.random.default_rng(seed)
    yield (rng.standard_normal(n) * 0.02).astype(np.float32)
    yield (rng.standard_normal(n) * 3.0).astype(np.float32)
    yield np.zeros(n, np.float32)
    yield np.full(n, 0.37, np.float32)
    yield np.full(n, -0.37, np.float32)
    x = (rng.standard_normal(n) * 0.02).astype(np.float32)
    x[::7] = 0.0
    x[::13] = -x[::13]
    yield x
    yield rng.integers(-5, 6, size=n).astype(np.float32) * np.float32(0.125)


@pytest.mark.parametrize("fmt", list(CASES))
def test_numpy_quantizer_matches_oracle(orc, fmt):
    n = 256 * 64
    for i, x in enumerate(_inputs(9, n)):
        a = quant.quantize(fmt, x)
        b = orc.quantize(CASES[fmt], x)
        assert a.dtype == np.uint8 and a.shape == b.shape
        bad = np.nonzero(a != b)[0]
        assert bad.size == 0, "input %d: first differing byte %d" % (i, bad[0])


def test_synthetic_weights_shape():
    w = quant.synthetic_weights("q4_k", 10, 512, seed=1)
    assert w.size == 10 * quant.row_bytes("q4_k", 512)
