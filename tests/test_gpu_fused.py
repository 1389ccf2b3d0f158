"""GPU parity of the neighbour fusions: the RMSNorm / SwiGLU activation prologues
of the decode matmuls (cri_matmul_rmsnorm, cri_matmul_swiglu) against the oracle's
unfused composition (orc_rmsnorm_residual / orc_silu_mul, then the reference's
dequant + sequential matmul), and the standalone cri_rmsnorm_residual /
cri_silu_mul.

Bars: matmul outputs ||C - C_ref||_inf <= 1e-5 ||C_ref||_inf (the M <= 16 bar);
hidden_out bit-exact (one fp32 add); the elementwise outputs 2e-6 normwise."""
import numpy as np
import pytest

from conftest import normwise_rel_err

torch = pytest.importorskip("torch")
import cretif_amd as cri  # noqa: E402
from cretif_amd import quant  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-5
EW_TOL = 2e-6
FMTS = ["q8_0", "q4_0", "q5_0", "q4_k", "q6_k", "fp16"]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rnd(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


# (M, N, K): M = 1 runs the GEMV (skinny for Q4_K), 2..16 the skinny kernel (Q4_K, Q6_K) or the
# element-wise kernel, K = 4096 / 8192 at M = 16 gives the skinny kernel 2 / 4 activation chunks
# (1, 300, 8192) and (2, 256, 4096): two activation items per thread in the skinny kernel;
# (8, 256, 8192), (16, 128, 8192): the SwiGLU path splits the chunks over two workgroups
SHAPES = [(1, 512, 2048), (2, 300, 2048), (7, 256, 1024), (16, 512, 2048), (16, 256, 4096), (16, 128, 8192),
          (1, 300, 8192), (2, 256, 4096), (8, 256, 8192)]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_matmul_rmsnorm(orc, fmt, M, N, K):
    W = quant.synthetic_weights(fmt, N, K, seed=M + N)
    h, r, w = rnd((M, K), 1 + M), rnd((M, K), 2 + M, 0.5), rnd(K, 3)
    dh, dr, dw, dW = dev(h), dev(r), dev(w), dev(W)
    hout = torch.full((M, K), float("nan"), device="cuda")
    C = torch.full((M, N), float("nan"), device="cuda")
    cri.matmul_rmsnorm(fmt, dh, dr, dw, hout, dW, C, M, N, K, 1e-5)
    out_ref, normed = orc.rmsnorm_residual(h, r, w, 1e-5)
    ref = orc.matmul_quant(fmt, normed, W, N, K)
    assert np.array_equal(host(hout), out_ref)
    assert normwise_rel_err(host(C), ref) <= TOL


@pytest.mark.parametrize("fmt", ["q4_k", "q8_0", "q6_k"])
@pytest.mark.parametrize("M", [1, 5])
def test_matmul_rmsnorm_no_residual_no_hidden_out(orc, fmt, M):
    N, K = 256, 2048
    W = quant.synthetic_weights(fmt, N, K, seed=11)
    h, w = rnd((M, K), 12, 3.0), rnd(K, 13)
    C = torch.empty(M, N, device="cuda")
    cri.matmul_rmsnorm(fmt, dev(h), None, dev(w), None, dev(W), C, M, N, K, 1e-6)
    _, normed = orc.rmsnorm_residual(h, None, w, 1e-6)
    assert normwise_rel_err(host(C), orc.matmul_quant(fmt, normed, W, N, K)) <= TOL


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_matmul_swiglu_fused_gateup_buffer(orc, fmt, M, N, K):
    # gate and up are the two halves of one [M, 2K] gate/up output: ld = 2K
    W = quant.synthetic_weights(fmt, N, K, seed=M * 3 + N)
    gu = rnd((M, 2 * K), 21 + M, 2.0)
    dgu = dev(gu)
    C = torch.full((M, N), float("nan"), device="cuda")
    cri.matmul_swiglu(fmt, dgu, dgu.data_ptr() + 4 * K, 2 * K, dev(W), C, M, N, K)
    act = orc.silu_mul(gu[:, :K], gu[:, K:])
    assert normwise_rel_err(host(C), orc.matmul_quant(fmt, act, W, N, K)) <= TOL


@pytest.mark.parametrize("fmt", ["q4_k", "q5_0"])
def test_matmul_swiglu_separate_buffers(orc, fmt):
    M, N, K = 4, 200, 2048
    W = quant.synthetic_weights(fmt, N, K, seed=31)
    g, u = rnd((M, K), 32, 3.0), rnd((M, K), 33)
    C = torch.empty(M, N, device="cuda")
    cri.matmul_swiglu(fmt, dev(g), dev(u), K, dev(W), C, M, N, K)
    assert normwise_rel_err(host(C), orc.matmul_quant(fmt, orc.silu_mul(g, u), W, N, K)) <= TOL


@pytest.mark.parametrize("fmt,offset", [("q4_k", 2), ("q8_0", 2), ("q4_k", 4)])
def test_misaligned_weights(orc, fmt, offset):
    # 2 bytes off: the element-wise kernel; Q4_K 4 bytes off (dword but not 16-byte
    # aligned): the batch-1 GEMV with the RMSNorm prologue
    M, N, K = 1, 64, 512
    W = quant.synthetic_weights(fmt, N, K, seed=41)
    buf = torch.zeros(W.size + 8, dtype=torch.uint8, device="cuda")
    buf[offset:offset + W.size] = dev(W)
    h, w = rnd((M, K), 42), rnd(K, 43)
    C = torch.empty(M, N, device="cuda")
    cri.matmul_rmsnorm(fmt, dev(h), None, dev(w), None, buf.data_ptr() + offset, C, M, N, K, 1e-5)
    _, normed = orc.rmsnorm_residual(h, None, w, 1e-5)
    assert normwise_rel_err(host(C), orc.matmul_quant(fmt, normed, W, N, K)) <= TOL


def test_prefill_batch_rejected():
    x = torch.zeros(17, 256, device="cuda")
    W = dev(quant.synthetic_weights("q4_k", 16, 256, seed=1))
    with pytest.raises(cri.CretifError) as e:
        cri.matmul_swiglu("q4_k", x, x, 256, W, torch.empty(17, 16, device="cuda"), 17, 16, 256)
    assert e.value.status == -5


@pytest.mark.parametrize("rows,n", [(1, 2048), (16, 2048), (5, 77), (2, 8192)])
def test_rmsnorm_residual_standalone(orc, rows, n):
    x, r, w = rnd((rows, n), 51), rnd((rows, n), 52), rnd(n, 53)
    dx = dev(x)
    normed = torch.empty(rows, n, device="cuda")
    cri.rmsnorm_residual(dx, dev(r), dev(w), dx, normed, rows, n, 1e-5)  # in place, as the reference calls it
    out_ref, n_ref = orc.rmsnorm_residual(x, r, w, 1e-5)
    assert np.array_equal(host(dx), out_ref)
    assert normwise_rel_err(host(normed), n_ref) <= EW_TOL


def test_silu_mul_standalone(orc):
    g, u = rnd(100003, 61, 4.0), rnd(100003, 62)
    dg = dev(g)
    cri.silu_mul(dg, dev(u), dg, g.size)  # out aliasing gate
    assert normwise_rel_err(host(dg), orc.silu_mul(g, u)) <= EW_TOL
