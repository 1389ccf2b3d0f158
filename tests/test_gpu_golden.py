"""The HIP path, through the C ABI, against the committed golden vectors
(tests/golden/path_vectors.npz; the oracle's outputs on the reference's test generators).
Bars as in the other parity tests: dequantisation bit-exact; matmuls with M <= 16 and the fp32
neighbours ||C - C_ref||_inf <= 1e-5 ||C_ref||_inf; prefill (M > 16, fp16 operands on the
matrix cores) 1e-3; attention 1e-5; rmsnorm's residual sum bit-exact and its normed row and
silu_mul at 2e-6."""
import os

import numpy as np
import pytest

from conftest import bits_equal, normwise_rel_err

torch = pytest.importorskip("torch")
import cretif_amd as cri  # noqa: E402

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "path_vectors.npz")
FMTS = ["q8_0", "q4_0", "q5_0", "q4_k", "q6_k", "fp16"]
BE = {"q8_0": 32, "q4_0": 32, "q5_0": 32, "q4_k": 256, "q6_k": 256}


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN) as z:
        return {k: z[k] for k in z.files}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q5_0", "q4_k", "q6_k"])
def test_golden_dequant(g, fmt):
    N, K, _ = (int(x) for x in g["shape_NK"])
    out = torch.full((N * K,), float("nan"), device="cuda")
    cri.dequantize(fmt, dev(g[fmt + "_B"]), out, N * K // BE[fmt])
    assert bits_equal(host(out), g[fmt + "_deq"])


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M", [1, 2, 3, 5, 16, 17, 20])
def test_golden_matmul(g, fmt, M):
    N, K, _ = (int(x) for x in g["shape_NK"])
    C = torch.full((M, N), float("nan"), device="cuda")
    cri.matmul(fmt, dev(g["A"][:M]), dev(g[fmt + "_B"]), C, M, N, K)
    tol = 1e-5 if M <= 16 else 1e-3
    assert normwise_rel_err(host(C), g[fmt + "_C"][:M]) <= tol


def test_golden_transposed_b(g):
    M, N, K = (int(x) for x in g["tb_shape"])
    C = torch.full((M, N), float("nan"), device="cuda")
    cri.matmul_transposed_b(dev(g["tb_A"]), dev(g["tb_B"]), C, M, N, K)
    assert normwise_rel_err(host(C), g["tb_C"]) <= 1e-5


@pytest.mark.parametrize("j", [0, 1])
def test_golden_gqa(g, j):
    H, Hkv, M, K, N = (int(x) for x in g["gqa%d_shape" % j])
    C = torch.full((H, M, N), float("nan"), device="cuda")
    cri.batched_matmul_gqa(dev(g["gqa%d_A" % j]), dev(g["gqa%d_B" % j]), C, H, Hkv, M, N, K)
    assert normwise_rel_err(host(C), g["gqa%d_C" % j]) <= 1e-5


def test_golden_attention(g):
    H, Hkv, D, T, L = (int(x) for x in g["att_shape"])
    out = torch.full((H * D,), float("nan"), device="cuda")
    cri.fused_decode_attention(dev(g["att_Q"]), dev(g["att_K"]), dev(g["att_V"]), out, H, Hkv, D, L,
                               float(g["att_scale"][0]))
    assert normwise_rel_err(host(out), g["att_out"]) <= 1e-5


def test_golden_elementwise(g):
    rows, n = g["rms_x"].shape
    out = torch.full((rows, n), float("nan"), device="cuda")
    normed = torch.full((rows, n), float("nan"), device="cuda")
    cri.rmsnorm_residual(dev(g["rms_x"]), dev(g["rms_r"]), dev(g["rms_w"]), out, normed, rows, n, 1e-5)
    assert bits_equal(host(out), g["rms_out"])
    assert normwise_rel_err(host(normed), g["rms_normed"]) <= 2e-6
    s = torch.full((g["silu_g"].size,), float("nan"), device="cuda")
    cri.silu_mul(dev(g["silu_g"]), dev(g["silu_u"]), s, g["silu_g"].size)
    assert normwise_rel_err(host(s), g["silu_out"]) <= 2e-6
