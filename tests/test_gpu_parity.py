"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Bars (from the path's contract):
  * dequantisation: bit-exact;
  * fused matmul / GEMV in fp32 FMA: ||C - C_ref||_inf <= 1e-5 * ||C_ref||_inf;
  * prefill (M > 16) on the fp16-operand MFMA GEMM: the same norm, 1e-3;
  * exact-integer inputs (every partial sum exact): bit-exact for every format
    and every kernel variant, whatever the summation order.
"""
import numpy as np
import pytest

from conftest import bits_equal, normwise_rel_err

torch = pytest.importorskip("torch")
import cretif_amd as cri  # noqa: E402
from cretif_amd import quant  # noqa: E402

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5
PREFILL_TOL = 1e-3   # M > 16: fp16 operands, fp32 accumulation on the matrix cores
PREFILL_MIN_M = 17


def tol_for(M):
    return GEMV_TOL if M < PREFILL_MIN_M else PREFILL_TOL
FMTS = ["q8_0", "q4_0", "q5_0", "q4_k", "q6_k", "fp16"]
BE = {"q8_0": 32, "q4_0": 32, "q5_0": 32, "q4_k": 256, "q6_k": 256, "fp16": 1}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def weights(fmt, N, K, seed):
    return quant.synthetic_weights(fmt, N, K, seed=seed)


def run_matmul(fmt, A, Bq, N, K):
    M = A.shape[0]
    dA, dB = dev(A), dev(Bq)
    dC = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    cri.matmul(fmt, dA, dB, dC, M, N, K)
    return host(dC)


# ------------------------------------------------------------------ dequant
@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q6_k", "q4_k"])
def test_dequant_reference_blocks(orc, fmt):
    nb = 64 if fmt in ("q8_0", "q4_0") else 8  # ref:tests/test_dequantize.cu:214-416
    blocks = orc.make_blocks(fmt, nb)
    n = nb * BE[fmt]
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    cri.dequantize(fmt, dev(blocks), out, nb)
    assert bits_equal(host(out), orc.dequantize(fmt, blocks, n))


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q5_0", "q6_k", "q4_k"])
@pytest.mark.parametrize("nb", [1, 3, 257, 20000])
def test_dequant_random_bytes(orc, fmt, nb):
    rng = np.random.default_rng(nb)
    bb = quant.BLOCK_BYTES[fmt]
    raw = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    specials = np.array([0.0, -0.0, 2.0**-24, 3 * 2.0**-20, 0.02, -1.5, 65504.0], np.float16)
    d = rng.choice(specials, size=nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
    if fmt == "q6_k":
        raw[:, 208:210] = d
    else:
        raw[:, 0:2] = d
        if fmt == "q4_k":
            raw[:, 2:4] = rng.choice(specials, size=nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
    n = nb * BE[fmt]
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    cri.dequantize(fmt, dev(raw.ravel()), out, nb)
    assert bits_equal(host(out), orc.dequantize(fmt, raw.ravel(), n))


def test_dequant_q5_0_reference_roundtrip(orc):
    # ref:tests/test_matmul_quant.cu:569-603 (16 blocks from the LCG generator)
    x = orc.random_matrix_lcg(1, 16 * 32, seed=42).ravel()
    blocks = orc.quantize("q5_0", x)
    out = torch.empty(512, dtype=torch.float32, device="cuda")
    cri.dequantize_q5_0(dev(blocks), out, 16)
    assert bits_equal(host(out), orc.dequantize("q5_0", blocks, 512))


# ------------------------------------------------------------------ GEMV (M = 1)
GEMV_SHAPES = [
    ("q8_0", 1536, 576),     # BASELINE config 1 (SmolLM2-135M FFN up-proj)
    ("q8_0", 8192, 2048),
    ("q8_0", 2048, 8192),
    ("q4_0", 8192, 2048),    # config 2
    ("q4_0", 2048, 8192),
    ("q5_0", 8192, 2048),
    ("q5_0", 2048, 8192),
    ("q4_k", 2048, 2048),    # config 3
    ("q4_k", 512, 2048),
    ("q4_k", 8192, 2048),
    ("q4_k", 2048, 8192),
    ("q6_k", 2048, 2048),
    ("q6_k", 512, 2048),
    ("q6_k", 128256, 2048),  # Llama-3.2-1B lm_head
    ("fp16", 8192, 2048),
    ("fp16", 2048, 8192),
    ("fp16", 576, 576),
]


@pytest.mark.parametrize("fmt,N,K", GEMV_SHAPES)
def test_gemv_baseline_shapes(orc, fmt, N, K):
    A = quant.randn(K, seed=2000 + K).reshape(1, K)
    Bq = weights(fmt, N, K, seed=1000 + N)
    got = run_matmul(fmt, A, Bq, N, K)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    err = normwise_rel_err(got, ref)
    assert err <= GEMV_TOL, err


# ragged row counts on the 512-thread workgroups (plain GEMVs at the 2048-wave budget: Q8_0, or
# K >= 4096), including a last workgroup that is only partly used
@pytest.mark.parametrize("fmt,N,K", [("q8_0", 5001, 2048), ("q8_0", 4097, 1024), ("q4_k", 4099, 4096),
                                     ("q4_0", 2053, 8192), ("q5_0", 3001, 4096), ("q6_k", 2051, 8192),
                                     ("fp16", 2049, 4096)])
def test_gemv_wide_workgroups_ragged(orc, fmt, N, K):
    A = quant.randn(K, seed=3 * K + N).reshape(1, K)
    Bq = weights(fmt, N, K, seed=N + 11 * K)
    got = run_matmul(fmt, A, Bq, N, K)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    assert normwise_rel_err(got, ref) <= GEMV_TOL


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("N", [1, 3, 17, 130, 1001])
@pytest.mark.parametrize("K", [256, 768, 4096, 16384])
def test_gemv_ragged(orc, fmt, N, K):
    A = quant.randn(K, seed=K + N).reshape(1, K)
    Bq = weights(fmt, N, K, seed=N * 7 + K)
    got = run_matmul(fmt, A, Bq, N, K)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    assert normwise_rel_err(got, ref) <= GEMV_TOL


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q5_0", "fp16"])
@pytest.mark.parametrize("K", [32, 96, 320, 576 + 32])
def test_gemv_k_not_multiple_of_64(orc, fmt, K):
    # odd block counts per row: rows not dword aligned -> element-wise path
    N = 77
    A = quant.randn(K, seed=K).reshape(1, K)
    Bq = weights(fmt, N, K, seed=K + 1)
    got = run_matmul(fmt, A, Bq, N, K)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    assert normwise_rel_err(got, ref) <= GEMV_TOL


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M", [1, 2, 5, 16])
def test_exact_integer_bit_exact(orc, fmt, M):
    from test_oracle_matmul import exact_case

    N, K = 300, 1024
    A, Bq = exact_case(fmt, M, N, K, seed=M)
    got = run_matmul(fmt, A, Bq, N, K)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    assert bits_equal(got, ref)


@pytest.mark.parametrize("offset,N,K", [(2, 64, 512), (4, 300, 2048), (8, 1001, 4096)])
def test_misaligned_weight_pointer(orc, offset, N, K):
    # B starting `offset` bytes into an allocation: 2 bytes routes around the
    # dword-aligned vector loads (element-wise kernel); 4 or 8 bytes is dword
    # aligned but not 16-byte aligned, which the skinny kernel needs, so Q4_K at
    # M = 1 runs the batch-1 GEMV
    A = quant.randn(K, seed=1).reshape(1, K)
    Bq = weights("q4_k", N, K, seed=2)
    buf = torch.zeros(Bq.size + offset, dtype=torch.uint8, device="cuda")
    buf[offset:] = dev(Bq)
    C = torch.empty(1, N, dtype=torch.float32, device="cuda")
    cri.matmul_q4_k(dev(A), buf.data_ptr() + offset, C, 1, N, K)
    ref = orc.matmul_quant("q4_k", A, Bq, N, K)
    assert normwise_rel_err(host(C), ref) <= GEMV_TOL


# ------------------------------------------------------------------ M > 1
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,N,K", [(4, 64, 256), (2, 200, 512), (16, 512, 2048), (33, 70, 768)])
def test_matmul_small_m(orc, fmt, M, N, K):
    A = quant.randn(M * K, seed=M * 31 + K).reshape(M, K)
    Bq = weights(fmt, N, K, seed=N + K)
    got = run_matmul(fmt, A, Bq, N, K)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    assert normwise_rel_err(got, ref) <= tol_for(M)


# Shapes chosen for the skinny kernel's activation-staging and row-layout paths
# (K % 256 == 0, 1 <= M <= 16): activation chunk KC = largest multiple of 256
# dividing K with M * KC <= 32768; items = M * KC / 8 against 512 threads.
SKINNY_PATH_SHAPES = [
    (1, 300, 8192),    # paired rows, two activation items per thread (1024)
    (2, 300, 4096),    # paired rows, two items per thread (1024)
    (3, 300, 4096),    # paired rows, general staging loop (1536 items)
    (8, 300, 4096),    # largest paired M, general staging (4096 items)
    (9, 300, 4096),    # smallest unpaired M: KC 2048, 2 chunks, eight items per thread
    (12, 300, 2048),   # unpaired, one chunk of eight items per thread
    (16, 300, 8192),   # FFN-down-like: 4 chunks of eight items per thread
    (16, 300, 16384),  # 8 chunks
    (16, 40000, 4096),  # 2 chunks and more row groups than workgroups (grid stride)
    # chunks split over two workgroups adding into a zero-filled C (few row groups, even chunk count)
    (5, 300, 8192),    # paired rows, KC 4096: one chunk per workgroup
    (8, 300, 8192),    # largest paired M, one chunk per workgroup
    (16, 2048, 8192),  # the FFN down shape: 128 row groups, two chunks per workgroup
    (16, 4096, 8192),  # 256 row groups: not split
]


@pytest.mark.parametrize("fmt", ["q4_k", "q6_k", "q8_0"])
@pytest.mark.parametrize("M,N,K", SKINNY_PATH_SHAPES)
def test_skinny_staging_paths(orc, fmt, M, N, K):
    A = quant.randn(M * K, seed=M * 131 + K + N).reshape(M, K)
    Bq = weights(fmt, N, K, seed=N + 3 * K + M)
    got = run_matmul(fmt, A, Bq, N, K)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    assert normwise_rel_err(got, ref) <= GEMV_TOL


@pytest.mark.parametrize("fmt,N,K", [(f, n, k) for f in ("q8_0", "q4_0", "q5_0")
                                     for n, k in ((1536, 576), (300, 2048), (17, 4096), (1001, 64), (8192, 2048))]
                         + [("q6_k", 2048, 2048), ("q6_k", 300, 4096), ("q6_k", 17, 256)])
def test_two_row_gemv(orc, fmt, N, K):
    # M = 2 of Q8_0 / Q4_0 / Q5_0 / Q6_K with K <= 4096 (K % 64 == 0): one GEMV launch
    # multiplies each decoded weight unit with both activation rows
    A = quant.randn(2 * K, seed=N + K).reshape(2, K)
    Bq = weights(fmt, N, K, seed=N * 3 + K)
    got = run_matmul(fmt, A, Bq, N, K)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    assert normwise_rel_err(got, ref) <= GEMV_TOL
    # each row alone through the batch-1 GEMV gives the same bits, unless the batch-1 GEMV
    # takes two units per lane there (Q4_0, Q5_0, Q4_K at K = 2048 from 8192 rows) or is the
    # K-sliced GEMV, which adds in another order (Q4_K at K in {1024, 2048, 4096, 8192}, Q8_0,
    # Q4_0 and Q5_0 at K = 8192)
    sliced = (fmt == "q4_k" and K in (1024, 2048, 4096, 8192)) or (fmt in ("q8_0", "q4_0", "q5_0") and K == 8192)
    if not (sliced or (fmt in ("q4_0", "q5_0", "q4_k") and K == 2048 and N >= 8192)):
        for m in range(2):
            assert np.array_equal(run_matmul(fmt, A[m:m + 1], Bq, N, K), got[m:m + 1])


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q5_0"])
@pytest.mark.parametrize("M,N,K", [(3, 1536, 576), (5, 300, 320), (16, 77, 4032), (7, 1001, 64),
                                   (3, 300, 2048), (4, 8192, 2048)])
def test_row_pair_gemv(orc, fmt, M, N, K):
    # row pairs of the two-row GEMV, one per grid row (an odd M repeats its last row in the
    # last pair, unstored): 3 <= M <= 4, and up to 16 when K % 256 != 0 (no skinny kernel)
    A = quant.randn(M * K, seed=M * 7 + K).reshape(M, K)
    Bq = weights(fmt, N, K, seed=N + M + K)
    got = run_matmul(fmt, A, Bq, N, K)
    assert normwise_rel_err(got, orc.matmul_quant(fmt, A, Bq, N, K)) <= GEMV_TOL
    # the batch-1 GEMV gives each row's bits where it is the same kernel family (see above)
    sliced = (fmt == "q4_k" and K in (1024, 2048, 4096, 8192)) or (fmt in ("q8_0", "q4_0", "q5_0") and K == 8192)
    if not (sliced or (fmt in ("q4_0", "q5_0", "q4_k") and K == 2048 and N >= 8192)):
        for m in (0, M - 1):
            assert np.array_equal(run_matmul(fmt, A[m:m + 1], Bq, N, K), got[m:m + 1])


@pytest.mark.parametrize("fmt", ["q4_k", "q8_0"])
def test_skinny_chunk_split_is_deterministic(fmt):
    # M <= 8: two partial sums per output added atomically in either order, the same bits
    # every call
    M, N, K = 5, 2048, 8192
    A = quant.randn(M * K, seed=91).reshape(M, K)
    Bq = weights(fmt, N, K, seed=92)
    first = run_matmul(fmt, A, Bq, N, K)
    for _ in range(3):
        assert np.array_equal(run_matmul(fmt, A, Bq, N, K), first)


@pytest.mark.parametrize("fmt", ["q4_k", "q8_0"])
def test_skinny_many_splits_differ_only_in_order(orc, fmt):
    # M > 8 without a workspace (the bare C ABI): K split over 16 workgroups whose fp32
    # partial sums are added atomically, so calls may differ in the last bits -- by no more
    # than a reordering of 16 terms can (the decode step passes a workspace and gets a fixed
    # order: its replay test checks bit equality)
    M, N, K = 16, 2048, 8192
    A = quant.randn(M * K, seed=91).reshape(M, K)
    Bq = weights(fmt, N, K, seed=92)
    first = run_matmul(fmt, A, Bq, N, K)
    assert normwise_rel_err(first, orc.matmul_quant(fmt, A, Bq, N, K)) <= GEMV_TOL
    for _ in range(3):
        assert normwise_rel_err(run_matmul(fmt, A, Bq, N, K), first) <= 16 * 2.0 ** -24


@pytest.mark.parametrize("M", [2, 7, 16])
def test_q6_k_skinny_lm_head_rows(orc, M):
    # decode batches against a slice of the lm_head shape (full-range int8 sub-scales)
    N, K = 4096, 2048
    A = quant.randn(M * K, seed=M + 77).reshape(M, K)
    Bq = weights("q6_k", N, K, seed=78)
    got = run_matmul("q6_k", A, Bq, N, K)
    ref = orc.matmul_quant("q6_k", A, Bq, N, K)
    assert normwise_rel_err(got, ref) <= GEMV_TOL


@pytest.mark.parametrize("off", [2, 4, 6])
def test_q6_k_skinny_unaligned(orc, off):
    # 210-byte super-blocks at 2-byte offsets; K/256 odd so rows alternate alignment
    M, N, K = 5, 37, 768
    A = quant.randn(M * K, seed=off).reshape(M, K)
    Bq = weights("q6_k", N, K, seed=off + 1)
    buf = torch.zeros(Bq.size + 8, dtype=torch.uint8, device="cuda")
    buf[off:off + Bq.size] = dev(Bq)
    C = torch.empty(M, N, dtype=torch.float32, device="cuda")
    cri.matmul_q6_k(dev(A), buf.data_ptr() + off, C, M, N, K)
    assert normwise_rel_err(host(C), orc.matmul_quant("q6_k", A, Bq, N, K)) <= GEMV_TOL


@pytest.mark.parametrize("K", [256, 768, 2048])
@pytest.mark.parametrize("off", [0, 4])
def test_q6_k_prefill_super_block_alignments(orc, K, off):
    # the register-decode prefill kernel copies 210-byte super-blocks that start 0 or 2 bytes past
    # a dword boundary (odd super-blocks; alternate rows when K/256 is odd); N odd puts the
    # buffer's last super-block on either alignment, and the weights end where the buffer does
    M, N = 40, 33
    A = quant.randn(M * K, seed=K + off).reshape(M, K)
    Bq = weights("q6_k", N, K, seed=K + off + 1)
    buf = torch.zeros(Bq.size + off, dtype=torch.uint8, device="cuda")
    buf[off:] = dev(Bq)
    C = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    cri.matmul_q6_k(dev(A), buf.data_ptr() + off, C, M, N, K)
    assert normwise_rel_err(host(C), orc.matmul_quant("q6_k", A, Bq, N, K)) <= PREFILL_TOL


@pytest.mark.parametrize("fmt", ["q4_0", "q5_0", "q8_0", "fp16"])
@pytest.mark.parametrize("off", [0, 2, 4])
@pytest.mark.parametrize("N", [33, 64])
def test_prefill_block_alignments(orc, fmt, off, N):
    # the register-decode prefill kernel reads 18 / 22 / 34-byte blocks (FP16: each lane's 64
    # bytes of a step) from dword-aligned rows (offsets 0 and 4; 4 is not 16-byte aligned); at
    # offset 2 the rows are not dword-aligned and the element-wise kernel takes the product.  The
    # weights end where the buffer does.
    M, K = 40, 512
    A = quant.randn(M * K, seed=N + off).reshape(M, K)
    Bq = weights(fmt, N, K, seed=N + off + 1)
    buf = torch.zeros(Bq.size + off, dtype=torch.uint8, device="cuda")
    buf[off:] = dev(Bq)
    C = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    cri.matmul(fmt, dev(A), buf.data_ptr() + off, C, M, N, K)
    assert normwise_rel_err(host(C), orc.matmul_quant(fmt, A, Bq, N, K)) <= PREFILL_TOL


def test_reference_test_shapes(orc):
    # shapes and LCG data of ref:tests/test_matmul_quant.cu (MatmulQ8_0/Q4_0/Q4_K/Q5_0/Q6_K/FP16)
    cases = [
        ("q8_0", 4, 64, 128, 1, 2), ("q8_0", 1, 576, 576, 10, 20), ("q4_0", 4, 64, 128, 3, 4),
        ("q4_k", 4, 32, 256, 5, 6), ("q5_0", 4, 64, 128, 7, 8), ("q5_0", 1, 576, 576, 11, 12),
        ("q6_k", 4, 32, 256, 10, 11), ("q6_k", 1, 576, 1536, 20, 21), ("q4_k", 1, 1536, 512, 30, 31),
        ("fp16", 4, 256, 256, 100, 101), ("fp16", 1, 576, 576, 102, 103), ("fp16", 1, 576, 1536, 104, 105),
        ("fp16", 4, 576, 576, 106, 107),
    ]
    for fmt, M, N, K, sa, sb in cases:
        A = orc.random_matrix_lcg(M, K, seed=sa)
        B = orc.random_matrix_lcg(N, K, seed=sb)
        Bq = B.astype(np.float16).view(np.uint8).ravel() if fmt == "fp16" else orc.quantize(fmt, B)
        got = run_matmul(fmt, A, Bq, N, K)
        ref = orc.matmul_quant(fmt, A, Bq, N, K)
        assert normwise_rel_err(got, ref) <= GEMV_TOL, (fmt, M, N, K)


# ------------------------------------------------------------------ prefill (M > 16): MFMA GEMM
PREFILL_SHAPES = [(17, 64, 256), (64, 130, 512), (128, 128, 2048), (130, 300, 768), (200, 1000, 1024),
                  (512, 256, 2048)]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,N,K", PREFILL_SHAPES)
def test_prefill_matches_oracle(orc, fmt, M, N, K):
    A = quant.randn(M * K, seed=M * 13 + K).reshape(M, K)
    Bq = weights(fmt, N, K, seed=N * 3 + K)
    got = run_matmul(fmt, A, Bq, N, K)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    err = normwise_rel_err(got, ref)
    assert err <= PREFILL_TOL, err


@pytest.mark.parametrize("fmt", ["q8_0", "q4_k", "q6_k", "q4_0", "q5_0", "fp16"])
@pytest.mark.parametrize("N,K", [(8192, 2048), (2048, 8192)])
def test_prefill_baseline_config(orc, fmt, N, K):
    # 512 tokens x Llama-3.2-1B FFN gate/up and down, every output against the oracle (its
    # columns split over host threads), and every 64 x 256 tile on its own: a tile-mapping or
    # split-k error in any one tile fails
    M = 512
    A = quant.randn(M * K, seed=K).reshape(M, K)
    Bq = weights(fmt, N, K, seed=N)
    got = run_matmul(fmt, A, Bq, N, K)
    ref = orc.matmul_quant_mt(fmt, A, Bq, N, K)
    assert normwise_rel_err(got, ref) <= PREFILL_TOL
    for m0 in range(0, M, 64):
        for n0 in range(0, N, 256):
            t = (slice(m0, m0 + 64), slice(n0, n0 + 256))
            assert normwise_rel_err(got[t], ref[t]) <= PREFILL_TOL, (m0, n0)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M", [17, 64, 130])
def test_prefill_exact_integer_bit_exact(orc, fmt, M):
    # integer activations and power-of-two-scaled integer weights are exact in
    # fp16 and every fp32 partial sum is exact: the MFMA GEMM must be bit-exact
    from test_oracle_matmul import exact_case

    N, K = 300, 1024
    A, Bq = exact_case(fmt, M, N, K, seed=M)
    got = run_matmul(fmt, A, Bq, N, K)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    assert bits_equal(got, ref)


@pytest.mark.parametrize("fmt", ["q8_0", "q4_k", "q6_k", "q4_0", "q5_0", "fp16"])
@pytest.mark.parametrize("M,N,K", [(64, 128, 8192), (40, 100, 4096), (33, 64, 16384)])
def test_prefill_split_k(orc, fmt, M, N, K):
    # few output tiles: the k range is split over workgroups and added with atomics
    A = quant.randn(M * K, seed=M + K).reshape(M, K)
    Bq = weights(fmt, N, K, seed=N + 5)
    got = run_matmul(fmt, A, Bq, N, K)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    assert normwise_rel_err(got, ref) <= PREFILL_TOL


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q5_0", "fp16"])
@pytest.mark.parametrize("K", [576, 96, 32 * 35])
def test_prefill_k_32_multiples(orc, fmt, K):
    # K = 576 (SmolLM2, 9 steps of 64) takes the MFMA GEMM; K an odd multiple of
    # 32 takes the element-wise kernel
    M, N = 40, 1536
    A = quant.randn(M * K, seed=K + 3).reshape(M, K)
    Bq = weights(fmt, N, K, seed=K + 4)
    got = run_matmul(fmt, A, Bq, N, K)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    assert normwise_rel_err(got, ref) <= PREFILL_TOL


@pytest.mark.parametrize("fmt", ["q8_0", "q4_k"])
def test_prefill_unaligned_output(orc, fmt):
    # C one float into an allocation (not 16-byte aligned) and N not a multiple
    # of 4: scalar stores
    M, N, K = 48, 257, 512
    A = quant.randn(M * K, seed=9).reshape(M, K)
    Bq = weights(fmt, N, K, seed=10)
    buf = torch.full((M * N + 1,), float("nan"), dtype=torch.float32, device="cuda")
    cri.matmul(fmt, dev(A), dev(Bq), buf.data_ptr() + 4, M, N, K)
    got = host(buf)[1:].reshape(M, N)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    assert normwise_rel_err(got, ref) <= PREFILL_TOL


def test_prefill_large_activations(orc):
    # activations up to ~3e3 (well inside fp16) keep the relative bound
    M, N, K = 64, 256, 2048
    A = quant.randn(M * K, seed=11).reshape(M, K) * 1000.0
    Bq = weights("q8_0", N, K, seed=12)
    got = run_matmul("q8_0", A, Bq, N, K)
    ref = orc.matmul_quant("q8_0", A, Bq, N, K)
    assert normwise_rel_err(got, ref) <= PREFILL_TOL


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q5_0", "q4_k", "q6_k", "fp16", "q8_0_k576"])
@pytest.mark.parametrize("case", ["huge", "tiny", "mixed"])
def test_prefill_activation_range(orc, fmt, case):
    # fp16 holds |x| < 65504, and rows of very small values only as subnormals: rows of
    # activations ~1e5 (inf in fp16) or ~1e-7 must still meet the bar, each row against its own
    # norm; 'mixed' puts such rows among ordinary ones (and into a split-k launch).  Every format
    # with K % 256 == 0 runs the register-decode prefill kernel, q8_0 at K = 576 the LDS-staged
    # one; both flag such rows and recompute them in fp32.
    M, N, K = (64, 300, 2048) if case != "mixed" else (40, 128, 8192)
    if fmt == "q8_0_k576":
        fmt, K = "q8_0", 576
    A = quant.randn(M * K, seed=17).reshape(M, K)
    if case == "huge":
        A *= 1e5
    elif case == "tiny":
        A *= 1e-7
    else:
        A[3] *= 1e5
        A[21] *= 3e-8
        A[39, 100] = 7e4
    Bq = weights(fmt, N, K, seed=18)
    got = run_matmul(fmt, A, Bq, N, K)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    assert np.all(np.isfinite(got))
    for r in range(M):
        assert normwise_rel_err(got[r], ref[r]) <= PREFILL_TOL, (r, normwise_rel_err(got[r], ref[r]))


def test_k_zero_writes_zeros():
    C = torch.full((3, 5), 7.0, device="cuda")
    A = torch.zeros(3, 1, device="cuda")
    B = torch.zeros(64, dtype=torch.uint8, device="cuda")
    cri.matmul_q8_0(A, B, C, 3, 5, 0)
    assert np.all(host(C) == 0.0)


def test_nondefault_stream(orc):
    N, K = 1024, 2048
    A = quant.randn(K, seed=9).reshape(1, K)
    Bq = weights("q4_k", N, K, seed=10)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        dA, dB = dev(A), dev(Bq)
        C = torch.empty(1, N, device="cuda")
        cri.matmul_q4_k(dA, dB, C, 1, N, K, stream=s)
    s.synchronize()
    assert normwise_rel_err(C.cpu().numpy(), orc.matmul_quant("q4_k", A, Bq, N, K)) <= GEMV_TOL


# ------------------------------------------------------------------ fp32 neighbours
@pytest.mark.parametrize("M,N,K", [(1, 4, 3), (2, 4, 3), (64, 64, 64), (1, 5000, 2048), (3, 1000, 2048),
                                   (1, 333, 100), (16, 4096, 2048), (2, 64, 16), (5, 1001, 3072), (16, 77, 4096),
                                   (4, 100, 100), (17, 300, 256)])
def test_transposed_b(orc, M, N, K):
    A = quant.randn(M * K, seed=M + K).reshape(M, K)
    B = quant.randn(N * K, seed=N + K).reshape(N, K)
    C = torch.empty(M, N, device="cuda")
    cri.matmul_transposed_b(dev(A), dev(B), C, M, N, K)
    assert normwise_rel_err(host(C), orc.matmul_transposed_b(A, B)) <= GEMV_TOL


def test_transposed_b_tied_head_batch16():
    # the tied LM head at decode batch 16 (ref:src/embedding.cu:85-135): 128256 x 2048 fp32
    # streamed once through the fp32 matrix cores, against a float64 product
    M, N, K = 16, 128256, 2048
    rng = np.random.default_rng(21)
    A = rng.standard_normal((M, K), dtype=np.float32)
    B = (rng.standard_normal((N, K), dtype=np.float32) * 0.02).astype(np.float32)
    C = torch.empty(M, N, device="cuda")
    cri.matmul_transposed_b(dev(A), dev(B), C, M, N, K)
    ref = A.astype(np.float64) @ B.astype(np.float64).T
    got = host(C)
    assert normwise_rel_err(got, ref) <= GEMV_TOL
    for r in (0, 7, 15):
        assert normwise_rel_err(got[r], ref[r]) <= GEMV_TOL


@pytest.mark.parametrize("H,Hkv,M,N,K", [
    (4, 2, 2, 3, 4),          # ref:tests/test_attention.cu:389-423
    (32, 8, 1, 2048, 64),     # decode Q K^T, kv = 2048
    (32, 8, 1, 64, 2048),     # decode P V
    (32, 8, 16, 2048, 64),
    (32, 8, 16, 64, 2048),
    (6, 3, 5, 37, 45),
    (8, 8, 3, 10, 700),
    (32, 8, 40, 1500, 300),   # matrix cores: 160 rows per KV head (ragged row tile), ragged n, k stages
    (4, 1, 7, 90, 1030),      # split kernel: ragged k stage, 28 rows
    (32, 8, 512, 64, 512),    # prefill P V (ref:src/attention.cu:837-861): matrix cores
    (32, 8, 512, 512, 64),    # prefill Q K^T: matrix cores
    (8, 2, 70, 100, 36),      # matrix cores: R = 280, N = 100, K = 36 (a partial k stage)
    (8, 4, 33, 8, 8),         # matrix cores: one partial tile each way, K = 8 (< one stage)
    (4, 2, 40, 4, 4),         # matrix cores: the smallest K and N
    (4, 1, 32, 64, 300),      # matrix cores, long-K variant: partial last stage, stage count padded
    (8, 2, 40, 102, 36),      # N % 4 != 0: the split kernel
])
def test_gqa(orc, H, Hkv, M, N, K):
    A = quant.randn(H * M * K, seed=H + M).reshape(H, M, K)
    B = quant.randn(Hkv * K * N, seed=N + K).reshape(Hkv, K, N)
    C = torch.empty(H, M, N, device="cuda")
    cri.batched_matmul_gqa(dev(A), dev(B), C, H, Hkv, M, N, K)
    ref = orc.batched_matmul_gqa(A, B, H, Hkv, M, N, K)
    assert normwise_rel_err(host(C), ref) <= GEMV_TOL


# ---- the 32-element formats and FP16 on the skinny MFMA kernel (2 <= M <= 16) ----
def random_code_weights(fmt, N, K, seed):
    """Raw random bytes for every quant field (all codes, Q8_0 -128 included, all Q5_0
    high bits), with each block's fp16 scale replaced by a finite value in
    [2^-10, 2^3]; FP16 weights as random finite halves."""
    rng = np.random.default_rng(seed)
    if fmt == "fp16":
        return rng.uniform(-2, 2, size=N * K).astype(np.float16).view(np.uint8)
    bb = quant.BLOCK_BYTES[fmt]
    raw = rng.integers(0, 256, size=(N * K // 32, bb), dtype=np.uint8)
    d = (rng.choice([-1.0, 1.0], size=raw.shape[0]) * 2.0 ** rng.uniform(-10, 3, size=raw.shape[0])).astype(np.float16)
    raw[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    return raw.ravel()


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q5_0", "fp16"])
@pytest.mark.parametrize("M,N,K,off", [(2, 37, 256, 0), (3, 200, 768, 4), (9, 64, 2048, 8), (16, 50, 8192, 12),
                                       (16, 1024, 4096, 0)])
def test_skinny_block_formats_random_codes(orc, fmt, M, N, K, off):
    A = quant.randn(M * K, seed=M * 7 + K).reshape(M, K)
    Bq = random_code_weights(fmt, N, K, seed=N + off)
    buf = torch.zeros(Bq.size + 16, dtype=torch.uint8, device="cuda")
    buf[off:off + Bq.size] = dev(Bq)
    C = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    cri.matmul(fmt, dev(A), buf.data_ptr() + off, C, M, N, K)
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    assert normwise_rel_err(host(C), ref) <= GEMV_TOL


@pytest.mark.parametrize("n_bytes", [16, 4096 * 16 + 16, 9437184])
def test_stream_read_probe(n_bytes):
    # the bandwidth probe writes nothing but the sink: a zero buffer leaves it untouched; a
    # buffer whose first word is the probe's constant (the rest zero) sets it, since the
    # thread that reads word 0 reads three other, zero, chunks with it (n_bytes >= 16 KB)
    src = torch.zeros(n_bytes, dtype=torch.uint8, device="cuda")
    sink = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    cri.stream_read(src, n_bytes, sink)
    assert int(host(sink)[0]) == 7
    if n_bytes >= 16 * 1024:
        src.view(torch.int32)[0] = int(np.uint32(0x9E3779B9).view(np.int32))
        cri.stream_read(src, n_bytes, sink)
        assert np.uint32(host(sink)[0]) == np.uint32(0x9E3779B9)


# ------------------------------------------------------------------ cri_matmul_ws
@pytest.mark.parametrize("fmt", ["q4_k", "q8_0", "q6_k", "q4_0"])
@pytest.mark.parametrize("M,N,K", [(16, 2048, 8192), (12, 512, 4096), (9, 300, 8192), (5, 256, 2048), (2, 1024, 2048)])
def test_matmul_ws_same_bits_every_call(orc, fmt, M, N, K):
    # 2..16 rows with a workspace: the K split's partial sums are added in split order, so three
    # calls give the same bits (the atomic path of cri_matmul need not), within the bar of the oracle
    A = quant.randn(M * K, seed=M + N + K).reshape(M, K)
    Bq = weights(fmt, N, K, seed=N + K)
    need = cri.matmul_workspace_bytes(fmt, M, N, K)
    assert need > 0
    ws = torch.empty(need // 4, dtype=torch.float32, device="cuda")
    dA, dB = dev(A), dev(Bq)
    outs = []
    for _ in range(3):
        C = torch.full((M, N), float("nan"), device="cuda")
        cri.matmul_ws(fmt, dA, dB, C, M, N, K, ws)
        outs.append(host(C))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    assert normwise_rel_err(outs[0], orc.matmul_quant(fmt, A, Bq, N, K)) <= GEMV_TOL


@pytest.mark.parametrize("fmt", ["q4_k", "q8_0", "fp16"])
@pytest.mark.parametrize("M,N,K,splits", [(96, 2048, 2048, 4), (64, 512, 8192, 16), (17, 300, 4096, 8)])
def test_matmul_ws_prefill_split(orc, fmt, M, N, K, splits):
    # above 16 rows with few output tiles the prefill GEMM splits K over workgroups: with a
    # workspace the partial sums are stored there and added in split order (the same bits on
    # every call), without one they go to C with atomics; both within the prefill bar of the oracle
    A = quant.randn(M * K, seed=M + N + K).reshape(M, K)
    Bq = weights(fmt, N, K, seed=N + K + 1)
    need = cri.matmul_workspace_bytes(fmt, M, N, K)
    assert need == splits * M * N * 4
    ws = torch.full((need // 4,), float("nan"), dtype=torch.float32, device="cuda")
    dA, dB = dev(A), dev(Bq)
    outs = []
    for _ in range(3):
        C = torch.full((M, N), float("nan"), device="cuda")
        cri.matmul_ws(fmt, dA, dB, C, M, N, K, ws)
        outs.append(host(C))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    ref = orc.matmul_quant(fmt, A, Bq, N, K)
    err = normwise_rel_err(outs[0], ref)
    C = torch.full((M, N), float("nan"), device="cuda")
    cri.matmul(fmt, dA, dB, C, M, N, K)
    err_atomic = normwise_rel_err(host(C), ref)
    print("prefill split %s %dx%dx%d: workspace %.2e, atomics %.2e" % (fmt, M, N, K, err, err_atomic))
    assert err <= PREFILL_TOL and err_atomic <= PREFILL_TOL
    # the two differ only in the order the partial sums are added (a few fp32 roundings)
    assert normwise_rel_err(outs[0], host(C)) <= 1e-5
    # where the workspace is used, C must be 16-byte aligned and N a multiple of 4
    wide = torch.empty(M, N + 4, device="cuda")
    with pytest.raises(cri.CretifError):
        cri.matmul_ws(fmt, dA, dB, wide.view(-1)[1:1 + M * N], M, N, K, ws)
    with pytest.raises(cri.CretifError):  # too small
        cri.matmul_ws(fmt, dA, dB, C, M, N, K, ws, need - 16)


def test_matmul_ws_errors_and_other_row_counts(orc):
    fmt, N, K = "q4_k", 512, 2048
    A = quant.randn(16 * K, seed=3).reshape(16, K)
    Bq = weights(fmt, N, K, seed=4)
    need = cri.matmul_workspace_bytes(fmt, 16, N, K)
    ws = torch.empty(need // 4, dtype=torch.float32, device="cuda")
    C = torch.empty(16, N, device="cuda")
    with pytest.raises(cri.CretifError):  # too small
        cri.matmul_ws(fmt, dev(A), dev(Bq), C, 16, N, K, ws, need - 16)
    with pytest.raises(cri.CretifError):  # none at all
        cri.matmul_ws(fmt, dev(A), dev(Bq), C, 16, N, K, None)
    wide = torch.empty(16, N + 4, device="cuda")
    with pytest.raises(cri.CretifError):  # C 4 bytes past a 16-byte boundary
        cri.matmul_ws(fmt, dev(A), dev(Bq), wide.view(-1)[1:1 + 16 * N], 16, N, K, ws)
    with pytest.raises(cri.CretifError):  # N not a multiple of 4
        cri.matmul_ws(fmt, dev(A), dev(Bq), C, 16, N - 2, K, ws)
    with pytest.raises(cri.CretifError):
        cri.matmul_ws(9, dev(A), dev(Bq), C, 16, N, K, ws)
    # one row, and a prefill-sized batch whose tiles fill the GPU unsplit, use no workspace (null
    # is fine) and match cri_matmul; a prefill-sized batch with few tiles splits K and needs one
    assert cri.matmul_workspace_bytes(fmt, 1, N, K) == 0 and cri.matmul_workspace_bytes(fmt, 512, 8192, K) == 0
    assert cri.matmul_workspace_bytes(fmt, 17, N, K) == 4 * 17 * N * 4
    with pytest.raises(cri.CretifError):
        cri.matmul_ws(fmt, dev(A), dev(Bq), torch.empty(17, N, device="cuda"), 17, N, K, None)
    for M in (1,):
        Am = quant.randn(M * K, seed=M).reshape(M, K)
        C1 = torch.empty(M, N, device="cuda")
        cri.matmul_ws(fmt, dev(Am), dev(Bq), C1, M, N, K, None)
        assert normwise_rel_err(host(C1), orc.matmul_quant(fmt, Am, Bq, N, K)) <= tol_for(M)
