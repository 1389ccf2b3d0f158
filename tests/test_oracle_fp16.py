"""Pin the oracle's IEEE binary16 codec against numpy's (an independent implementation)."""
import numpy as np


def test_half_to_float_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.half_to_float(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_float_to_half_rne(orc):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    # plus every tie / boundary neighbourhood of the half grid
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    h = h[np.isfinite(h)]
    mids = []
    for delta in (-1, 0, 1):
        hb = h.view(np.uint32).astype(np.int64)
        mids.append((hb + (1 << 12) + delta).astype(np.uint32).view(np.float32))  # near halfway to next half
    special = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, -65520.0, 2.0**-24, 2.0**-25, 2.0**-25 * 1.0001,
                        3 * 2.0**-26, 6.1035156e-05, np.inf, -np.inf, 1e-45, 0.1, 0.02], np.float32)
    f = np.concatenate([f] + mids + [special])
    f = f[~np.isnan(f)]
    got = orc.float_to_half(f)
    ref = f.astype(np.float16).view(np.uint16)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, "first mismatch: %r -> %#06x vs numpy %#06x" % (f[bad[0]], got[bad[0]], ref[bad[0]])


def test_float_to_half_nan_stays_nan(orc):
    f = np.array([np.nan, -np.nan], np.float32)
    back = orc.half_to_float(orc.float_to_half(f))
    assert np.all(np.isnan(back))
