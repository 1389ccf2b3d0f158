"""Pins the oracle's decode-step neighbours: orc_rope
(ref:src/kernels/elementwise.cu:232-257), orc_argmax (ref:src/embedding.cu:155-200)
and the decode-step composition (ref:src/model.cu:876-1039) built from pinned
functions.  CPU only."""
import numpy as np
import pytest

from cretif_amd import quant


def f64_rope(x, pos, head_dim, n_heads, theta):
    x = np.asarray(x, np.float64).reshape(n_heads, head_dim // 2, 2)
    i = np.arange(head_dim // 2)
    ang = pos * theta ** (-2.0 * i / head_dim)
    c, s = np.cos(ang), np.sin(ang)
    y = np.empty_like(x)
    y[..., 0] = x[..., 0] * c - x[..., 1] * s
    y[..., 1] = x[..., 0] * s + x[..., 1] * c
    return y.ravel()


def test_rope_position_zero_is_identity(orc):
    x = np.random.default_rng(1).standard_normal(32 * 64).astype(np.float32)
    assert np.array_equal(orc.rope(x, 0, 64, 32, 500000.0), x)


@pytest.mark.parametrize("pos", [1, 7, 100, 2047])
def test_rope_against_f64_rotation(orc, pos):
    H, D, theta = 8, 64, 10000.0
    x = np.random.default_rng(pos).standard_normal(H * D).astype(np.float32)
    got = orc.rope(x, pos, D, H, theta)
    ref = f64_rope(x, pos, D, H, theta)
    # the fp32 angle pos * freq is within pos * 2^-24 of the exact one; cos/sin add ~1 ulp
    tol = 4.0 * (pos * 2.0 ** -24 + 2.0 ** -23) * np.max(np.abs(x)) * 2
    assert np.max(np.abs(got - ref)) <= tol
    # each (2i, 2i+1) pair keeps its length
    gp, xp = got.reshape(-1, 2).astype(np.float64), x.reshape(-1, 2).astype(np.float64)
    np.testing.assert_allclose(np.hypot(gp[:, 0], gp[:, 1]), np.hypot(xp[:, 0], xp[:, 1]), rtol=1e-6)


def test_rope_pair_zero_turns_by_pos_radians(orc):
    # pair 0 has frequency theta^0 = 1 exactly, so its angle is pos itself
    x = np.zeros(64, np.float32)
    x[0] = 1.0
    got = orc.rope(x, 3, 64, 1, 10000.0)
    assert abs(got[0] - np.cos(3.0)) < 2e-7 and abs(got[1] - np.sin(3.0)) < 2e-7


def test_rope_composes_as_rotations(orc):
    H, D = 4, 64
    x = np.random.default_rng(9).standard_normal(H * D).astype(np.float32)
    two = orc.rope(orc.rope(x, 5, D, H, 10000.0), 11, D, H, 10000.0)
    one = orc.rope(x, 16, D, H, 10000.0)
    assert np.max(np.abs(two - one)) < 1e-5


def test_argmax_rules(orc):
    rng = np.random.default_rng(4)
    for n in (1, 7, 1000, 128256):
        x = rng.standard_normal(n).astype(np.float32)
        assert orc.argmax(x) == int(np.argmax(x))
    assert orc.argmax(np.array([1, 5, 5, 2], np.float32)) == 1          # ties: the first index
    assert orc.argmax(np.array([np.nan, 1, np.nan, 3], np.float32)) == 3  # NaN never wins
    assert orc.argmax(np.full(9, -np.inf, np.float32)) == 0
    assert orc.argmax(np.full(9, np.nan, np.float32)) == 0


def tiny_model(seed=0, tied=False, tok="q8_0"):
    dim, H, Hkv, D, F, V = 256, 4, 2, 64, 512, 300
    rng = np.random.default_rng(seed)

    def w(fmt, n, k, s):
        return fmt, quant.synthetic_weights(fmt, n, k, seed=s)

    layers = []
    for i in range(2):
        b = 100 * (seed + 1) + 10 * i
        layers.append({
            "attn_norm": (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32),
            "ffn_norm": (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32),
            "q": w("q4_k", H * D, dim, b), "k": w("q4_k", Hkv * D, dim, b + 1), "v": w("q6_k", Hkv * D, dim, b + 2),
            "o": w("q8_0", dim, H * D, b + 3), "gate": w("q4_k", F, dim, b + 4), "up": w("q4_k", F, dim, b + 5),
            "down": w("q5_0", dim, F, b + 6)})
    table = quant.synthetic_weights(tok, V, dim, seed=7) if tok != "fp32" else \
        rng.standard_normal(V * dim).astype(np.float32) * 0.02
    return {"n_heads": H, "n_kv_heads": Hkv, "head_dim": D, "dim": dim, "ffn": F, "vocab": V, "eps": 1e-5,
            "theta": 10000.0, "tok": (tok, table), "layers": layers,
            "out_norm": (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32),
            "lm": None if tied else ("q6_k", quant.synthetic_weights("q6_k", V, dim, seed=8))}


def fresh_cache(model, T, seed):
    rng = np.random.default_rng(seed)
    shape = (T, model["n_kv_heads"], model["head_dim"])
    return ([rng.standard_normal(shape).astype(np.float32) for _ in model["layers"]],
            [rng.standard_normal(shape).astype(np.float32) for _ in model["layers"]])


def test_step_batch_equals_one_token_at_a_time(orc):
    # causal rows: a batch of 3 tokens at pos gives, row by row, what three single-token steps give
    # (every per-row operation is the same sequential fp32 arithmetic), and writes the same cache
    m = tiny_model()
    ids, pos = [5, 17, 299], 9
    kb, vb = fresh_cache(m, 32, 1)
    batch, nb = orc.decode_step(m, ids, pos, kb, vb)
    ks, vs = fresh_cache(m, 32, 1)
    for t, i in enumerate(ids):
        one, n1 = orc.decode_step(m, [i], pos + t, ks, vs)
        assert np.array_equal(one[0], batch[t]) and n1[0] == nb[t]
    for a, b in zip(kb + vb, ks + vs):
        assert np.array_equal(a, b)


def test_step_appends_rotated_keys_and_plain_values(orc):
    m = tiny_model(seed=2, tied=True, tok="fp32")
    kc, vc = fresh_cache(m, 16, 2)
    before = [k.copy() for k in kc]
    orc.decode_step(m, [3, 4], 6, kc, vc)
    for k0, k1 in zip(before, kc):
        assert np.array_equal(k0[:6], k1[:6]) and np.array_equal(k0[8:], k1[8:])  # only rows 6, 7 change
        assert not np.array_equal(k0[6:8], k1[6:8])
