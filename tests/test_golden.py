"""The committed golden vectors (tests/golden/path_vectors.npz, written by
tests/golden/make_golden.py from the reference's test generators) on the CPU: the oracle
still reproduces every one bit for bit, and independent numpy restatements agree with them
(the loop-form dequantisers of ref:tests/test_dequantize.cu:23-131 bit-exactly, the products
within the fp32 rounding bound of an fp64 brute force)."""
import os

import numpy as np
import pytest

from conftest import bits_equal

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "path_vectors.npz")
FMTS = ["q8_0", "q4_0", "q5_0", "q4_k", "q6_k", "fp16"]


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN) as z:  # allow_pickle stays False
        return {k: z[k] for k in z.files}


def test_oracle_reproduces_every_vector(orc, g):
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(os.path.dirname(GOLDEN),
                                                                              "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    fresh = mg.build()
    assert sorted(fresh) == sorted(g)
    for k, v in fresh.items():
        assert v.dtype == g[k].dtype and v.shape == g[k].shape, k
        assert np.array_equal(v.view(np.uint8), g[k].view(np.uint8)), k


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q5_0", "q4_k", "q6_k"])
def test_dequant_vectors_match_loop_form(orc, g, fmt):
    if fmt == "q4_k":
        ref = orc.np_dequant_q4_k_loopform(g[fmt + "_B"])
    elif fmt == "q6_k":
        ref = orc.np_dequant_q6_k_loopform(g[fmt + "_B"])
    else:
        ref = orc.np_dequant_simple(fmt, g[fmt + "_B"])
    assert bits_equal(ref, g[fmt + "_deq"])


@pytest.mark.parametrize("fmt", FMTS)
def test_matmul_vectors_within_fp32_bound(orc, g, fmt):
    N, K, M = (int(x) for x in g["shape_NK"])
    if fmt == "fp16":
        W = g["fp16_B"].view(np.float16).astype(np.float64).reshape(N, K)
    else:
        W = g[fmt + "_deq"].astype(np.float64).reshape(N, K)
    A = g["A"].astype(np.float64)
    exact = A @ W.T
    gamma = K * 2.0**-24 / (1 - K * 2.0**-24)
    bound = gamma * (np.abs(A) @ np.abs(W).T)
    assert np.all(np.abs(g[fmt + "_C"] - exact) <= bound)
    # and not trivially: every row and column carries signal
    assert np.all(np.abs(exact).max(axis=1) > 0.1) and np.all(np.abs(exact).max(axis=0) > 0.1)


def test_neighbour_vectors_within_bound(g):
    a, b = g["tb_A"].astype(np.float64), g["tb_B"].astype(np.float64)
    K = a.shape[1]
    gamma = K * 2.0**-24 / (1 - K * 2.0**-24)
    assert np.all(np.abs(g["tb_C"] - a @ b.T) <= gamma * (np.abs(a) @ np.abs(b).T))
    for j in range(2):
        H, Hkv, M, K, N = (int(x) for x in g["gqa%d_shape" % j])
        A, B = g["gqa%d_A" % j].astype(np.float64), g["gqa%d_B" % j].astype(np.float64)
        gamma = K * 2.0**-24 / (1 - K * 2.0**-24)
        for h in range(H):
            kv = h // (H // Hkv)
            assert np.all(np.abs(g["gqa%d_C" % j][h] - A[h] @ B[kv]) <= gamma * (np.abs(A[h]) @ np.abs(B[kv])))


def test_attention_vector_vs_fp64(orc, g):
    H, Hkv, D, T, L = (int(x) for x in g["att_shape"])
    ref = orc.np_decode_attention_f64(g["att_Q"], g["att_K"], g["att_V"], H, Hkv, D, L, g["att_scale"][0])
    assert np.max(np.abs(g["att_out"] - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_elementwise_vectors_vs_fp64(g):
    x, r, w = (g[k].astype(np.float64) for k in ("rms_x", "rms_r", "rms_w"))
    assert bits_equal(g["rms_out"], (g["rms_x"] + g["rms_r"]))  # one fp32 add
    v = g["rms_out"].astype(np.float64)
    normed = v * w / np.sqrt((v * v).mean(axis=1, keepdims=True) + 1e-5)
    assert np.max(np.abs(g["rms_normed"] - normed)) <= 1e-6 * np.max(np.abs(normed))
    gg, u = g["silu_g"].astype(np.float64), g["silu_u"].astype(np.float64)
    ref = gg / (1 + np.exp(-gg)) * u
    assert np.max(np.abs(g["silu_out"] - ref)) <= 1e-6 * np.max(np.abs(ref))
