"""Pins the decode-attention oracle (oracle/oracle.c: orc_decode_attention,
orc_decode_attention_online) before the GPU kernel is compared against it.

The two functions restate the reference's two formulations (the CPU test's
two-pass softmax, ref:tests/test_attention.cu:972-1008 with cpu_softmax :110-122,
and the kernel's single-pass recurrence, ref:src/attention.cu:446-493); they are
checked against each other, against an fp64 numpy brute force, and against
closed forms that a wrong index, a dropped scale or a wrong GQA head mapping
would break."""
import numpy as np
import pytest

from conftest import normwise_rel_err

# (n_heads, n_kv_heads, head_dim, kv_len): the reference tests' shapes
# (ref:tests/test_attention.cu:1010-1130) plus Llama-3.2-1B at 2048 positions
SHAPES = [(1, 1, 8, 4), (4, 4, 16, 8), (8, 2, 16, 16), (4, 4, 64, 512), (32, 8, 64, 2048), (6, 3, 5, 77)]


def make(H, Hkv, D, T, seed, spread=1.0, extra=0):
    rng = np.random.default_rng(seed)
    Q = rng.standard_normal(H * D).astype(np.float32) * spread
    K = rng.standard_normal((T + extra) * Hkv * D).astype(np.float32) * spread
    V = rng.standard_normal((T + extra) * Hkv * D).astype(np.float32)
    return Q, K, V


@pytest.mark.parametrize("H,Hkv,D,T", SHAPES)
def test_two_formulations_agree(orc, H, Hkv, D, T):
    Q, K, V = make(H, Hkv, D, T, seed=H * 1000 + T)
    s = 1.0 / np.sqrt(D)
    a = orc.decode_attention(Q, K, V, H, Hkv, D, T, s)
    b = orc.decode_attention(Q, K, V, H, Hkv, D, T, s, online=True)
    assert normwise_rel_err(a, b) < 2e-6


@pytest.mark.parametrize("H,Hkv,D,T", SHAPES)
def test_fp64_brute_force(orc, H, Hkv, D, T):
    Q, K, V = make(H, Hkv, D, T, seed=7 + T, spread=1.5)
    s = 1.0 / np.sqrt(D)
    ref = orc.np_decode_attention_f64(Q, K, V, H, Hkv, D, T, s)
    for online in (False, True):
        got = orc.decode_attention(Q, K, V, H, Hkv, D, T, s, online=online)
        assert normwise_rel_err(got, ref) < 1e-5


def test_single_position_returns_v_row(orc):
    Q, K, V = make(4, 2, 16, 1, seed=3)
    out = orc.decode_attention(Q, K, V, 4, 2, 16, 1, 0.25).reshape(4, 16)
    v = V.reshape(1, 2, 16)[0]
    for h in range(4):
        assert np.array_equal(out[h], v[h // 2])
    out = orc.decode_attention(Q, K, V, 4, 2, 16, 1, 0.25, online=True).reshape(4, 16)
    for h in range(4):
        assert np.array_equal(out[h], v[h // 2])


def test_zero_scale_gives_mean_of_v(orc):
    # all scores equal -> uniform weights; a dropped scale factor would not give this
    H, Hkv, D, T = 8, 2, 16, 100
    Q, K, V = make(H, Hkv, D, T, seed=11)
    out = orc.decode_attention(Q, K, V, H, Hkv, D, T, 0.0).reshape(H, D)
    mean = V.reshape(T, Hkv, D).astype(np.float64).mean(axis=0)
    for h in range(H):
        np.testing.assert_allclose(out[h], mean[h // (H // Hkv)], rtol=0, atol=1e-6)


def test_dominant_position_selects_its_v_row(orc):
    # one position scores 200 above the rest: exp(-200) underflows in fp32, the
    # output is exactly that position's V row
    H, Hkv, D, T, hot = 4, 1, 8, 50, 17
    Q = np.zeros(H * D, np.float32)
    Q[::D] = 1.0  # q = e_0 for every head
    K = np.zeros((T, Hkv, D), np.float32)
    K[hot, 0, 0] = 200.0
    V = np.random.default_rng(5).standard_normal((T, Hkv, D)).astype(np.float32)
    for online in (False, True):
        out = orc.decode_attention(Q, K, V, H, Hkv, D, T, 1.0, online=online).reshape(H, D)
        for h in range(H):
            assert np.array_equal(out[h], V[hot, 0])


def test_gqa_head_mapping(orc):
    # heads 4g..4g+3 read KV head g (h / G), not h % n_kv_heads
    H, Hkv, D, T = 8, 2, 8, 20
    Q, K, V = make(H, Hkv, D, T, seed=13)
    out = orc.decode_attention(Q, K, V, H, Hkv, D, T, 0.5).reshape(H, D)
    k3 = K.reshape(T, Hkv, D)
    v3 = V.reshape(T, Hkv, D)
    for h in range(H):
        single = orc.decode_attention(Q.reshape(H, D)[h], np.ascontiguousarray(k3[:, h // 4]),
                                      np.ascontiguousarray(v3[:, h // 4]), 1, 1, D, T, 0.5)
        assert np.array_equal(out[h], single)


def test_position_permutation_invariance(orc):
    H, Hkv, D, T = 4, 2, 16, 300
    Q, K, V = make(H, Hkv, D, T, seed=17)
    perm = np.random.default_rng(1).permutation(T)
    Kp = K.reshape(T, -1)[perm].ravel()
    Vp = V.reshape(T, -1)[perm].ravel()
    a = orc.decode_attention(Q, K, V, H, Hkv, D, T, 0.3)
    b = orc.decode_attention(Q, Kp, Vp, H, Hkv, D, T, 0.3)
    assert normwise_rel_err(a, b) < 2e-6


def test_cache_longer_than_kv_len(orc):
    # positions >= kv_len (the rest of a max_seq_len cache) are never read
    H, Hkv, D, T = 4, 2, 16, 33
    Q, K, V = make(H, Hkv, D, T, seed=19, extra=31)
    a = orc.decode_attention(Q, K, V, H, Hkv, D, T, 0.25)
    K2, V2 = K.copy(), V.copy()
    K2[T * Hkv * D:] = np.nan
    V2[T * Hkv * D:] = np.nan
    b = orc.decode_attention(Q, K2, V2, H, Hkv, D, T, 0.25)
    assert np.array_equal(a, b)
