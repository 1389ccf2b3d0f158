"""Pin the oracle's matmuls (ref:tests/test_matmul_quant.cu:30-41,
ref:tests/test_embedding.cu:98-109, ref:tests/test_attention.cu:76-85, 399-407).

* fp64 brute force within the standard fp32 summation bound
  |C - C64| <= gamma_K * sum_k |a_k w_k|, gamma_K = K u / (1 - K u), u = 2^-24;
* exact-integer KATs: power-of-two scales and small integer activations make
  every partial sum an integer below 2^24, so C is exact in any order;
* one-hot activations select single dequantised weights exactly;
* GQA head mapping: KV head kv serves heads [kv*G, (kv+1)*G).
"""
import numpy as np
import pytest

from conftest import bits_equal

FMTS = ["q8_0", "q4_0", "q5_0", "q4_k", "q6_k", "fp16"]
U = 2.0**-24


def _weights(orc, fmt, N, K, seed):
    w = orc.randn(N * K, seed=seed, sigma=0.02)
    if fmt == "fp16":
        return w.astype(np.float16).view(np.uint8)
    return orc.quantize("q4_k_asym" if fmt == "q4_k" else fmt, w)


def _deq(orc, fmt, Bq, N, K):
    return orc.dequantize(fmt, Bq, N * K).reshape(N, K)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,N,K", [(1, 64, 512), (4, 32, 1024), (3, 17, 256)])
def test_fp64_bound(orc, fmt, M, N, K):
    A = orc.randn(M * K, seed=100 + M, sigma=1.0).reshape(M, K)
    Bq = _weights(orc, fmt, N, K, seed=200 + N)
    C = orc.matmul_quant(fmt, A, Bq, N, K)
    W = _deq(orc, fmt, Bq, N, K)
    C64 = orc.np_matmul_f64(A, W)
    gamma = K * U / (1 - K * U)
    bound = gamma * (np.abs(A).astype(np.float64) @ np.abs(W).astype(np.float64).T)
    assert np.all(np.abs(C - C64) <= bound + 1e-30)
    # and the fp32 result is the same as matmul_bt over the dequantised weights
    assert bits_equal(C, orc.matmul_bt(A, W))


def _exact_blocks(fmt, N, K, rng):
    """Weights whose dequantised values are small integers times a power of two."""
    nb = N * K // (32 if fmt in ("q8_0", "q4_0", "q5_0") else 256)
    if fmt == "q8_0":
        b = np.zeros((nb, 34), np.uint8)
        b[:, 0:2] = np.array([0.25], np.float16).view(np.uint8)
        b[:, 2:] = rng.integers(-20, 21, size=(nb, 32)).astype(np.int8).view(np.uint8)
    elif fmt == "q4_0":
        b = np.zeros((nb, 18), np.uint8)
        b[:, 0:2] = np.array([0.5], np.float16).view(np.uint8)
        b[:, 2:] = rng.integers(0, 256, size=(nb, 16))
    elif fmt == "q5_0":
        b = rng.integers(0, 256, size=(nb, 22)).astype(np.uint8)
        b[:, 0:2] = np.array([2.0], np.float16).view(np.uint8)
    elif fmt == "q4_k":
        b = rng.integers(0, 256, size=(nb, 144)).astype(np.uint8)
        b[:, 0:2] = np.array([0.125], np.float16).view(np.uint8)
        b[:, 2:4] = np.array([0.25], np.float16).view(np.uint8)
    elif fmt == "q6_k":
        b = rng.integers(0, 256, size=(nb, 210)).astype(np.uint8)
        b[:, 192:208] = rng.integers(-8, 9, size=(nb, 16)).astype(np.int8).view(np.uint8)
        b[:, 208:210] = np.array([0.0625], np.float16).view(np.uint8)
    else:  # fp16: small integers / 4
        return (rng.integers(-64, 65, size=N * K) / 4.0).astype(np.float16).view(np.uint8)
    return b.ravel()


def exact_case(fmt, M, N, K, seed):
    rng = np.random.default_rng(seed)
    Bq = _exact_blocks(fmt, N, K, rng)
    A = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    return A, Bq


@pytest.mark.parametrize("fmt", FMTS)
def test_exact_integer_kat(orc, fmt):
    M, N, K = 3, 40, 512
    A, Bq = exact_case(fmt, M, N, K, seed=42)
    W = _deq(orc, fmt, Bq, N, K).astype(np.float64)
    exact = A.astype(np.float64) @ W.T
    # every partial sum is an integer multiple of a power of two well inside 2^24 ulps
    assert np.max(np.abs(A).astype(np.float64) @ np.abs(W).T) < 2.0**20
    C = orc.matmul_quant(fmt, A, Bq, N, K)
    assert np.array_equal(C.astype(np.float64), exact)


@pytest.mark.parametrize("fmt", FMTS)
def test_one_hot_selects_weight(orc, fmt):
    N, K = 16, 512
    Bq = _weights(orc, fmt, N, K, seed=7)
    W = _deq(orc, fmt, Bq, N, K)
    ks = [0, 1, 31, 32, 255, 256, 511]
    A = np.zeros((len(ks), K), np.float32)
    for i, k in enumerate(ks):
        A[i, k] = 1.0
    C = orc.matmul_quant(fmt, A, Bq, N, K)
    assert bits_equal(C, W[:, ks].T)


def test_rows_subset_matches_full(orc):
    A = orc.randn(2 * 256, seed=1).reshape(2, 256)
    Bq = _weights(orc, "q4_k", 64, 256, seed=2)
    full = orc.matmul_quant("q4_k", A, Bq, 64, 256)
    part = orc.matmul_quant("q4_k", A, Bq, 64, 256, rows=(10, 30))
    assert bits_equal(part[:, 10:30], full[:, 10:30])


def test_transposed_b_fp64(orc):
    M, N, K = 5, 33, 300
    A = orc.randn(M * K, seed=1).reshape(M, K)
    B = orc.randn(N * K, seed=2).reshape(N, K)
    C = orc.matmul_transposed_b(A, B)
    gamma = K * U / (1 - K * U)
    bound = gamma * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64).T)
    assert np.all(np.abs(C - A.astype(np.float64) @ B.astype(np.float64).T) <= bound)


def test_gqa_mapping_and_fp64(orc):
    H, Hkv, M, N, K = 8, 2, 3, 20, 16
    A = orc.randn(H * M * K, seed=3).reshape(H, M, K)
    B = orc.randn(Hkv * K * N, seed=4).reshape(Hkv, K, N)
    C = orc.batched_matmul_gqa(A, B, H, Hkv, M, N, K)
    G = H // Hkv
    for h in range(H):
        ref = A[h].astype(np.float64) @ B[h // G].astype(np.float64)
        assert np.max(np.abs(C[h] - ref)) < 1e-5
    # distinct constant KV heads: head h must see kv = h // G exactly
    Bc = np.stack([np.full((K, N), kv + 1, np.float32) for kv in range(Hkv)])
    Ac = np.ones((H, M, K), np.float32)
    Cc = orc.batched_matmul_gqa(Ac, Bc, H, Hkv, M, N, K)
    for h in range(H):
        assert np.all(Cc[h] == K * (h // G + 1))


def test_gqa_reference_case(orc):
    # shape of ref:tests/test_attention.cu:389-423 (H=4, Hkv=2, M=2, N=3, K=4)
    A = orc.random_matrix_lcg(4 * 2, 4, seed=5).reshape(4, 2, 4)
    B = orc.random_matrix_lcg(2 * 4, 3, seed=6).reshape(2, 4, 3)
    C = orc.batched_matmul_gqa(A, B, 4, 2, 2, 3, 4)
    for h in range(4):
        assert np.allclose(C[h], A[h] @ B[h // 2], atol=1e-6)
