"""Writes tests/golden/path_vectors.npz: small input/output vectors for every function on
the path, computed by the CPU oracle (oracle/, pinned against the reference's known-answer
tests and closed forms by tests/test_oracle_*.py).  The weights and activations come from the
reference's own test generators (the LCG of ref:tests/test_matmul_quant.cu:187-195 and its host
quantizers, restated in oracle/oracle.c), so the vectors are the ones the reference's CPU
references would produce on its own test data.

Run from the repo root:  python tests/golden/make_golden.py
The committed file is checked by tests/test_golden.py (the oracle still reproduces it, on the
CPU) and tests/test_gpu_golden.py (the HIP path through the C ABI against it)."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as orc  # noqa: E402

FMTS = ["q8_0", "q4_0", "q5_0", "q4_k", "q6_k", "fp16"]
# 24 weight rows (not a multiple of the 16-row tiles), K = 512 (two K-quant super-blocks), up
# to 20 activation rows (batch-1 GEMV, row-pair GEMV, skinny MFMA and prefill paths)
N, K, M_MAX = 24, 512, 20
# matmul_transposed_b and GQA shapes: ragged, and one GQA case on the prefill (M >= 32) path
TB = (3, 40, 100)
GQA = [(4, 2, 3, 8, 5), (4, 1, 32, 16, 12)]
# decode attention: heads 4 / KV heads 2, head_dim 16, a cache of 20 rows read to kv_len 17
ATT = (4, 2, 16, 20, 17)


def weights(fmt, seed):
    w = orc.random_matrix_lcg(N, K, seed=seed)
    if fmt == "fp16":
        return orc.float_to_half(w).view(np.uint8).ravel()
    return orc.quantize(fmt, w)


def build():
    v = {"shape_NK": np.array([N, K, M_MAX], np.int32)}
    A = orc.random_matrix_lcg(M_MAX, K, seed=7)
    v["A"] = A
    for i, fmt in enumerate(FMTS):
        B = weights(fmt, 100 + i)
        v[fmt + "_B"] = B
        if fmt != "fp16":
            v[fmt + "_deq"] = orc.dequantize(fmt, B, N * K)
        # rows are independent: C[:M] is the M-row product for every M <= M_MAX
        v[fmt + "_C"] = orc.matmul_quant(fmt, A, B, N, K)

    M, Nt, Kt = TB
    a, b = orc.random_matrix_lcg(M, Kt, seed=11), orc.random_matrix_lcg(Nt, Kt, seed=12)
    v["tb_A"], v["tb_B"], v["tb_C"] = a, b, orc.matmul_transposed_b(a, b)
    v["tb_shape"] = np.array(TB, np.int32)

    for j, (H, Hkv, M, Kg, Ng) in enumerate(GQA):
        a = orc.random_matrix_lcg(H * M, Kg, seed=20 + j).reshape(H, M, Kg)
        b = orc.random_matrix_lcg(Hkv * Kg, Ng, seed=30 + j).reshape(Hkv, Kg, Ng)
        v["gqa%d_A" % j], v["gqa%d_B" % j] = a, b
        v["gqa%d_C" % j] = orc.batched_matmul_gqa(a, b, H, Hkv, M, Ng, Kg)
        v["gqa%d_shape" % j] = np.array([H, Hkv, M, Kg, Ng], np.int32)

    H, Hkv, D, T, L = ATT
    q = orc.random_matrix_lcg(1, H * D, seed=40).ravel()
    kc = orc.random_matrix_lcg(T, Hkv * D, seed=41)
    vc = orc.random_matrix_lcg(T, Hkv * D, seed=42)
    scale = np.float32(1.0) / np.float32(np.sqrt(np.float32(D)))
    v["att_Q"], v["att_K"], v["att_V"] = q, kc, vc
    v["att_out"] = orc.decode_attention(q, kc, vc, H, Hkv, D, L, scale, online=True)
    v["att_shape"] = np.array(ATT, np.int32)
    v["att_scale"] = np.array([scale], np.float32)

    x = orc.random_matrix_lcg(3, 96, seed=50)
    r = orc.random_matrix_lcg(3, 96, seed=51)
    w = orc.random_matrix_lcg(1, 96, seed=52).ravel()
    out, normed = orc.rmsnorm_residual(x, r, w, 1e-5)
    v["rms_x"], v["rms_r"], v["rms_w"], v["rms_out"], v["rms_normed"] = x, r, w, out, normed
    g = orc.random_matrix_lcg(1, 200, seed=53).ravel() * np.float32(8)
    u = orc.random_matrix_lcg(1, 200, seed=54).ravel()
    v["silu_g"], v["silu_u"], v["silu_out"] = g, u, orc.silu_mul(g, u)
    return v


def main():
    v = build()
    np.savez_compressed(os.path.join(HERE, "path_vectors.npz"), **v)
    print("wrote %d arrays, %d bytes of data" % (len(v), sum(a.nbytes for a in v.values())))


if __name__ == "__main__":
    main()
