"""Pin the oracle's dequantisers.

* reference KATs (ref:tests/test_dequantize.cu:250-279 and :317-344);
* index form (oracle.c, from ref:src/kernels/dequantize.cu) against the
  loop-form CPU references of ref:tests/test_dequantize.cu:23-131 restated
  separately in numpy -- a transposed index or swapped nibble in either fails;
* every code of every field, fp16 special scales;
* quantize -> dequantize round trips stay within the quantisation step
  (a wrong element order produces errors of the order of the block range).
"""
import numpy as np
import pytest

from conftest import bits_equal


def _q8_block(d, qs):
    b = np.zeros(34, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:] = np.asarray(qs, np.int8).view(np.uint8)
    return b


def test_kat_q8_0_single_block(orc):
    # ref:tests/test_dequantize.cu:250-279: d = 0.5, qs[i] = i - 16 -> 0.5 * (i - 16)
    out = orc.dequantize("q8_0", _q8_block(0.5, np.arange(32) - 16), 32)
    assert bits_equal(out, 0.5 * (np.arange(32, dtype=np.float32) - 16))


def test_kat_q4_0_all_0x88(orc):
    # ref:tests/test_dequantize.cu:317-344: d = 1, all nibbles 8 -> 0
    b = np.zeros(18, np.uint8)
    b[0:2] = np.array([1.0], np.float16).view(np.uint8)
    b[2:] = 0x88
    out = orc.dequantize("q4_0", b, 32)
    assert np.all(out == 0.0)


def test_kat_q4_0_element_order(orc):
    # Reference order: element i <- qs[i/2], low nibble for even i
    # (ref:src/kernels/dequantize.cu:87-97); GGML would put qs[j] low at j, high at j+16.
    b = np.zeros(18, np.uint8)
    b[0:2] = np.array([1.0], np.float16).view(np.uint8)
    b[2] = 0x19  # low nibble 9 -> element 0 = +1, high nibble 1 -> element 1 = -7
    b[3:] = 0x88
    out = orc.dequantize("q4_0", b, 32)
    assert out[0] == 1.0 and out[1] == -7.0 and np.all(out[2:] == 0.0)


@pytest.mark.parametrize("fmt,nb", [("q8_0", 64), ("q4_0", 64)])
def test_make_blocks_32(orc, fmt, nb):
    blocks = orc.make_blocks(fmt, nb)
    got = orc.dequantize(fmt, blocks, nb * 32)
    assert bits_equal(got, orc.np_dequant_simple(fmt, blocks))


def test_make_blocks_q6_k(orc):
    blocks = orc.make_blocks("q6_k", 8)
    got = orc.dequantize("q6_k", blocks, 8 * 256)
    assert bits_equal(got, orc.np_dequant_q6_k_loopform(blocks))


def test_make_blocks_q4_k(orc):
    blocks = orc.make_blocks("q4_k", 8)
    got = orc.dequantize("q4_k", blocks, 8 * 256)
    assert bits_equal(got, orc.np_dequant_q4_k_loopform(blocks))


def _random_blocks(fmt, nb, seed, d_choices=None):
    rng = np.random.default_rng(seed)
    bb = {"q8_0": 34, "q4_0": 18, "q5_0": 22, "q4_k": 144, "q6_k": 210}[fmt]
    raw = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    if d_choices is None:
        d_choices = np.array([0.0, -0.0, 2.0**-24, 2.0**-14 * 0.5, 6.1e-5, 0.02, 1.0, -3.5, 65504.0], np.float16)
    d = rng.choice(d_choices, size=nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
    if fmt == "q6_k":
        raw[:, 208:210] = d
    elif fmt == "q4_k":
        raw[:, 0:2] = d
        dm = rng.choice(d_choices, size=nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
        raw[:, 2:4] = dm
    else:
        raw[:, 0:2] = d
    return raw.ravel()


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q5_0", "q4_k", "q6_k"])
def test_random_bytes_both_forms(orc, fmt):
    """Random block bytes (every code of every field occurs) incl. fp16 specials as scales."""
    nb = 4096 if fmt in ("q8_0", "q4_0", "q5_0") else 1024
    blocks = _random_blocks(fmt, nb, seed=11)
    n = nb * (32 if fmt in ("q8_0", "q4_0", "q5_0") else 256)
    got = orc.dequantize(fmt, blocks, n)
    if fmt == "q6_k":
        ref = orc.np_dequant_q6_k_loopform(blocks)
    elif fmt == "q4_k":
        ref = orc.np_dequant_q4_k_loopform(blocks)
    else:
        ref = orc.np_dequant_simple(fmt, blocks)
    assert bits_equal(got, ref)


def test_q4_k_scale_min_codes(orc):
    """All 64 x 64 (sc, mn) codes of every sub-block through the 12-byte packing."""
    nb = 64 * 64
    blocks = np.zeros((nb, 144), np.uint8)
    blocks[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    blocks[:, 2:4] = np.array([1.0], np.float16).view(np.uint8)
    sc = np.repeat(np.arange(64), 64)
    mn = np.tile(np.arange(64), 64)
    s = np.zeros((nb, 12), np.int64)
    for j in range(4):  # same code for all 8 sub-blocks
        s[:, j] = (sc & 0x3F) | ((sc >> 4) << 6)
        s[:, j + 4] = (mn & 0x3F) | ((mn >> 4) << 6)
        s[:, j + 8] = (sc & 0x0F) | ((mn & 0x0F) << 4)
    blocks[:, 4:16] = s
    blocks[:, 16:] = 0x51  # nibble 1 (low), 5 (high)
    out = orc.dequantize("q4_k", blocks.ravel(), nb * 256).reshape(nb, 8, 32)
    for sb in range(8):
        nib = 1.0 if (sb % 2 == 0) else 5.0
        assert np.array_equal(out[:, sb, 0], sc * nib - mn), sb


def test_q6_k_all_codes(orc):
    """Every 6-bit code (ql nibble x qh pair) in every quarter, every int8 scale."""
    nb = 256
    blocks = np.zeros((nb, 210), np.uint8)
    blocks[:, 208:210] = np.array([1.0], np.float16).view(np.uint8)
    blocks[:, 192:208] = np.arange(256, dtype=np.uint8)[:, None]  # scale s (as int8) in every group
    codes = np.arange(64)
    for c in range(2):
        for l in range(32):
            code = codes[(l + 32 * c) % 64]
            lo, hi = code & 0xF, code >> 4
            blocks[:, 64 * c + l] = lo | (lo << 4)
            blocks[:, 64 * c + 32 + l] = lo | (lo << 4)
            blocks[:, 128 + 32 * c + l] = hi | (hi << 2) | (hi << 4) | (hi << 6)
    out = orc.dequantize("q6_k", blocks.ravel(), nb * 256).reshape(nb, 2, 4, 32)
    sc = np.arange(256, dtype=np.uint8).view(np.int8).astype(np.float64)
    for c in range(2):
        for l in range(32):
            code = codes[(l + 32 * c) % 64]
            for q in range(4):
                assert np.array_equal(out[:, c, q, l], sc * (code - 32)), (c, q, l)


ROUNDTRIP = {
    # bound on |x - dequant(quant(x))| relative to the block's max |x| (or range)
    "q8_0": 0.5 / 127 * 1.02 + 2.0**-10,
    "q4_0": 1.0 / 8 * 1.01 + 2.0**-9,   # +amax maps to +8 and clamps to +7: error up to one step
    "q5_0": 1.0 / 16 * 1.01 + 2.0**-9,
}


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q5_0"])
def test_roundtrip_32(orc, fmt):
    x = orc.randn(32 * 4096, seed=3, sigma=0.02)
    q = orc.quantize(fmt, x)
    y = orc.dequantize(fmt, q, x.size)
    amax = np.max(np.abs(x.reshape(-1, 32)), axis=1, keepdims=True)
    err = np.abs((y - x).reshape(-1, 32)) / amax
    assert err.max() <= ROUNDTRIP[fmt], err.max()


def test_roundtrip_q6_k(orc):
    x = orc.randn(256 * 1024, seed=4, sigma=0.02)
    y = orc.dequantize("q6_k", orc.quantize("q6_k", x), x.size)
    amax = np.max(np.abs(x.reshape(-1, 256)), axis=1, keepdims=True)
    err = np.abs((y - x).reshape(-1, 256)) / amax
    assert err.max() <= 0.02, err.max()
    assert np.median(err) < 0.01  # a misplaced element gives ~0.3


def test_roundtrip_q4_k_asym(orc):
    x = orc.randn(256 * 1024, seed=5, sigma=0.02)
    y = orc.dequantize("q4_k", orc.quantize("q4_k_asym", x), x.size)
    xb = x.reshape(-1, 256)
    rng = (xb.max(axis=1) - np.minimum(xb.min(axis=1), 0))[:, None]
    err = np.abs((y - x).reshape(-1, 256)) / rng
    assert err.max() <= 0.08, err.max()
    assert np.median(err) < 0.02


def test_roundtrip_q4_k_simple_nonneg(orc):
    # the reference's simplified Q4_K (dmin = 0) only represents non-negative values
    x = np.abs(orc.randn(256 * 256, seed=6, sigma=0.02))
    y = orc.dequantize("q4_k", orc.quantize("q4_k", x), x.size)
    amax = np.max(np.abs(x.reshape(-1, 256)), axis=1, keepdims=True)
    err = np.abs((y - x).reshape(-1, 256)) / amax
    assert err.max() <= 0.1, err.max()
