"""GPU parity of the fused decode attention (cretif_amd/csrc/attention.hip,
through cri_fused_decode_attention) against the CPU oracle's restatement of the
reference (orc_decode_attention: ref:tests/test_attention.cu:972-1008).

Bar: fp32 throughout, ||out - ref||_inf <= 1e-5 * ||ref||_inf (the reference's
own tests allow 1e-4 .. 2e-3 absolute); closed-form cases are exact."""
import numpy as np
import pytest

from conftest import normwise_rel_err

torch = pytest.importorskip("torch")
import cretif_amd as cri  # noqa: E402

pytestmark = pytest.mark.gpu

ATTN_TOL = 1e-5


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def make(H, Hkv, D, T, seed, spread=1.0, extra=0):
    rng = np.random.default_rng(seed)
    Q = rng.standard_normal(H * D).astype(np.float32) * spread
    K = rng.standard_normal((T + extra) * Hkv * D).astype(np.float32) * spread
    V = rng.standard_normal((T + extra) * Hkv * D).astype(np.float32)
    return Q, K, V


def run(Q, K, V, H, Hkv, D, T, scale, offset=0):
    """offset > 0 shifts every buffer by that many floats (unaligned vectors)."""
    def place(a):
        t = torch.empty(a.size + offset, dtype=torch.float32, device="cuda")
        t[offset:] = dev(a)
        return t, t.data_ptr() + 4 * offset
    (tq, pq), (tk, pk), (tv, pv) = place(Q), place(K), place(V)
    out = torch.full((H * D + offset,), float("nan"), dtype=torch.float32, device="cuda")
    cri.fused_decode_attention(pq, pk, pv, out.data_ptr() + 4 * offset, H, Hkv, D, T, scale)
    return host(out)[offset:]


SHAPES = [
    (1, 1, 8, 4), (4, 4, 16, 8), (8, 2, 16, 16), (4, 4, 64, 512),   # ref:tests/test_attention.cu:1010-1130
    (32, 8, 64, 2048),                                              # Llama-3.2-1B decode step
    (32, 8, 64, 1), (32, 8, 64, 63), (32, 8, 64, 65), (32, 8, 64, 4097),
    (32, 8, 128, 1000), (2, 1, 256, 300), (64, 8, 64, 700), (12, 4, 32, 129),
    (6, 3, 6, 77), (3, 3, 5, 100), (4, 2, 2, 50), (5, 5, 1, 9), (7, 1, 200, 31),
]


@pytest.mark.parametrize("H,Hkv,D,T", SHAPES)
def test_matches_oracle(orc, H, Hkv, D, T):
    Q, K, V = make(H, Hkv, D, T, seed=H * 7919 + D * 31 + T)
    s = 1.0 / np.sqrt(D)
    got = run(Q, K, V, H, Hkv, D, T, s)
    ref = orc.decode_attention(Q, K, V, H, Hkv, D, T, s)
    assert normwise_rel_err(got, ref) <= ATTN_TOL


@pytest.mark.parametrize("offset", [1, 2, 3])
@pytest.mark.parametrize("H,Hkv,D,T", [(32, 8, 64, 300), (8, 2, 16, 70)])
def test_unaligned_buffers(orc, H, Hkv, D, T, offset):
    Q, K, V = make(H, Hkv, D, T, seed=offset + T)
    got = run(Q, K, V, H, Hkv, D, T, 0.125, offset=offset)
    ref = orc.decode_attention(Q, K, V, H, Hkv, D, T, 0.125)
    assert normwise_rel_err(got, ref) <= ATTN_TOL


def test_cache_longer_than_kv_len(orc):
    # a max_seq_len cache: positions >= kv_len hold NaN and must never be read
    H, Hkv, D, T, extra = 32, 8, 64, 1000, 1048
    Q, K, V = make(H, Hkv, D, T, seed=23, extra=extra)
    K[T * Hkv * D:] = np.nan
    V[T * Hkv * D:] = np.nan
    got = run(Q, K, V, H, Hkv, D, T, 0.125)
    ref = orc.decode_attention(Q, K, V, H, Hkv, D, T, 0.125)
    assert np.all(np.isfinite(got))
    assert normwise_rel_err(got, ref) <= ATTN_TOL


def test_single_position_is_exact():
    H, Hkv, D = 32, 8, 64
    Q, K, V = make(H, Hkv, D, 1, seed=29)
    got = run(Q, K, V, H, Hkv, D, 1, 0.125).reshape(H, D)
    v = V.reshape(Hkv, D)
    for h in range(H):
        assert np.array_equal(got[h], v[h // 4])


def test_dominant_position_is_exact():
    H, Hkv, D, T, hot = 32, 8, 64, 2048, 1234
    Q = np.zeros(H * D, np.float32)
    Q[::D] = 1.0
    K = np.zeros((T, Hkv, D), np.float32)
    K[hot, :, 0] = 200.0
    V = np.random.default_rng(31).standard_normal((T, Hkv, D)).astype(np.float32)
    got = run(Q, K.ravel(), V.ravel(), H, Hkv, D, T, 1.0).reshape(H, D)
    for h in range(H):
        assert np.array_equal(got[h], V[hot, h // 4])


def test_large_scores_stay_finite(orc):
    # scores of order +-300: the running max keeps every exp in range.  An fp32
    # score this size carries ~3e-5 absolute rounding, which exp() turns into
    # relative weight errors of that order in any fp32 evaluation (the oracle's
    # included), so the bar here is the fp64 result, with the oracle's own
    # distance from it as the yardstick.
    H, Hkv, D, T = 32, 8, 64, 2048
    Q, K, V = make(H, Hkv, D, T, seed=37, spread=6.0)
    got = run(Q, K, V, H, Hkv, D, T, 1.0)
    exact = orc.np_decode_attention_f64(Q, K, V, H, Hkv, D, T, 1.0)
    ref_err = normwise_rel_err(orc.decode_attention(Q, K, V, H, Hkv, D, T, 1.0), exact)
    assert np.all(np.isfinite(got))
    assert normwise_rel_err(got, exact) <= 2 * ref_err + 1e-6


def test_zero_scale_gives_mean_of_v():
    H, Hkv, D, T = 32, 8, 64, 777
    Q, K, V = make(H, Hkv, D, T, seed=41)
    got = run(Q, K, V, H, Hkv, D, T, 0.0).reshape(H, D)
    mean = V.reshape(T, Hkv, D).astype(np.float64).mean(axis=0)
    for h in range(H):
        np.testing.assert_allclose(got[h], mean[h // 4], rtol=0, atol=2e-6)


def test_repeatable():
    # no atomics or workspace: the same inputs give the same bits every call
    H, Hkv, D, T = 32, 8, 64, 2048
    Q, K, V = make(H, Hkv, D, T, seed=43)
    a = run(Q, K, V, H, Hkv, D, T, 0.125)
    b = run(Q, K, V, H, Hkv, D, T, 0.125)
    assert np.array_equal(a, b)


def test_graph_replay(orc):
    H, Hkv, D, T = 32, 8, 64, 1500
    Q, K, V = make(H, Hkv, D, T, seed=47)
    dq, dk, dv = dev(Q), dev(K), dev(V)
    out = torch.zeros(H * D, device="cuda")
    ref = orc.decode_attention(Q, K, V, H, Hkv, D, T, 0.125)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        cri.fused_decode_attention(dq, dk, dv, out, H, Hkv, D, T, 0.125, stream=s)  # warm-up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        cri.fused_decode_attention(dq, dk, dv, out, H, Hkv, D, T, 0.125, stream=s)
    for _ in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert normwise_rel_err(host(out), ref) <= ATTN_TOL


# ---- split form with a caller workspace (cri_fused_decode_attention_ws) -------------
def run_ws(Q, K, V, H, Hkv, D, T, scale, ws_bytes=None):
    need = cri.decode_attention_workspace_size(H, Hkv, D, T)
    nbytes = need if ws_bytes is None else ws_bytes
    ws = torch.full((max(nbytes, 16) // 4 + 4,), float("nan"), dtype=torch.float32, device="cuda")
    out = torch.full((H * D,), float("nan"), dtype=torch.float32, device="cuda")
    cri.fused_decode_attention_ws(dev(Q), dev(K), dev(V), out, H, Hkv, D, T, scale, ws.data_ptr(), nbytes)
    return host(out)


WS_SHAPES = [
    (32, 8, 64, 2048), (32, 8, 64, 1), (32, 8, 64, 31), (32, 8, 64, 33), (32, 8, 64, 8191),
    (1, 1, 8, 4), (4, 4, 16, 8), (8, 2, 16, 16), (4, 4, 64, 512),   # reference test shapes
    (64, 8, 64, 700), (24, 4, 64, 300), (12, 2, 32, 129), (16, 16, 64, 1000), (32, 1, 64, 250), (8, 8, 4, 40),
]


@pytest.mark.parametrize("H,Hkv,D,T", WS_SHAPES)
def test_ws_matches_oracle(orc, H, Hkv, D, T):
    Q, K, V = make(H, Hkv, D, T, seed=H * 131 + T)
    s = 1.0 / np.sqrt(D)
    got = run_ws(Q, K, V, H, Hkv, D, T, s)
    ref = orc.decode_attention(Q, K, V, H, Hkv, D, T, s)
    assert normwise_rel_err(got, ref) <= ATTN_TOL


@pytest.mark.parametrize("records", [1, 2, 3, 7])
def test_ws_small_workspace(orc, records):
    # a workspace of `records` records per head: that many chunks (or fewer)
    H, Hkv, D, T = 32, 8, 64, 2048
    Q, K, V = make(H, Hkv, D, T, seed=records)
    got = run_ws(Q, K, V, H, Hkv, D, T, 0.125, ws_bytes=records * H * (D + 4) * 4)
    ref = orc.decode_attention(Q, K, V, H, Hkv, D, T, 0.125)
    assert normwise_rel_err(got, ref) <= ATTN_TOL


@pytest.mark.parametrize("H,Hkv,D,T", [(6, 3, 6, 77), (8, 2, 256, 90), (4, 2, 132, 50)])
def test_ws_other_shapes_use_workspace_free_kernel(H, Hkv, D, T):
    Q, K, V = make(H, Hkv, D, T, seed=D + T)
    a = run_ws(Q, K, V, H, Hkv, D, T, 0.2)
    b = run(Q, K, V, H, Hkv, D, T, 0.2)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("H,Hkv,D,T", [(32, 8, 128, 500), (8, 8, 96, 3000), (16, 4, 128, 1)])
def test_ws_head_dim_up_to_128(orc, H, Hkv, D, T):
    # head_dim 68..128 takes the split kernel's 8-slice layout
    Q, K, V = make(H, Hkv, D, T, seed=D + T)
    got = run_ws(Q, K, V, H, Hkv, D, T, 0.2)
    assert normwise_rel_err(got, orc.decode_attention(Q, K, V, H, Hkv, D, T, 0.2)) <= ATTN_TOL


def test_ws_dominant_position_is_exact():
    H, Hkv, D, T, hot = 32, 8, 64, 2048, 1999
    Q = np.zeros(H * D, np.float32)
    Q[::D] = 1.0
    K = np.zeros((T, Hkv, D), np.float32)
    K[hot, :, 0] = 200.0
    V = np.random.default_rng(53).standard_normal((T, Hkv, D)).astype(np.float32)
    got = run_ws(Q, K.ravel(), V.ravel(), H, Hkv, D, T, 1.0).reshape(H, D)
    for h in range(H):
        assert np.array_equal(got[h], V[hot, h // 4])


def test_ws_graph_replay(orc):
    H, Hkv, D, T = 32, 8, 64, 1500
    Q, K, V = make(H, Hkv, D, T, seed=59)
    dq, dk, dv = dev(Q), dev(K), dev(V)
    out = torch.zeros(H * D, device="cuda")
    ws = torch.empty(cri.decode_attention_workspace_size(H, Hkv, D, T) // 4, device="cuda")
    ref = orc.decode_attention(Q, K, V, H, Hkv, D, T, 0.125)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        cri.fused_decode_attention_ws(dq, dk, dv, out, H, Hkv, D, T, 0.125, ws, stream=s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        cri.fused_decode_attention_ws(dq, dk, dv, out, H, Hkv, D, T, 0.125, ws, stream=s)
    for _ in range(3):
        out.fill_(float("nan"))
        ws.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert normwise_rel_err(host(out), ref) <= ATTN_TOL


# ---- prompt attention (cri_prefill_attention): the reference's prefill flow, ref:src/attention.cu:809-871
def _oracle_rows(orc, q, kc, vc, H, Hkv, D, pos, scale):
    """Row m against the oracle's decode attention over positions [0, pos + m] (threads over rows)."""
    import concurrent.futures as cf

    with cf.ThreadPoolExecutor(8) as ex:
        rows = list(ex.map(lambda m: orc.decode_attention(q[m, :H * D], kc, vc, H, Hkv, D, pos + m + 1, scale),
                           range(q.shape[0])))
    return np.stack(rows)


@pytest.mark.parametrize("H,Hkv,D,M,pos", [(32, 8, 64, 17, 0), (32, 8, 64, 64, 100), (32, 8, 64, 512, 0),
                                           (32, 8, 64, 512, 1400), (32, 8, 64, 600, 37), (4, 2, 128, 100, 30),
                                           (8, 8, 32, 33, 5)])
def test_prefill_attention_matches_oracle(orc, H, Hkv, D, M, pos):
    # Q rows as the fused q/k/v projection leaves them (ldq = q + k + v widths); the cache rows past
    # pos + M hold NaN, which no product may read; 600 rows run as two row blocks (512 + 88)
    rng = np.random.default_rng(M + pos + D)
    ldq = H * D + 2 * Hkv * D
    q = rng.standard_normal((M, ldq)).astype(np.float32)
    T = pos + M + 40
    kc = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    vc = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    kc[pos + M:] = np.nan
    vc[pos + M:] = np.nan
    scale = 1.0 / np.sqrt(D)
    out = torch.full((M, H * D), float("nan"), device="cuda")
    cri.prefill_attention(dev(q), ldq, dev(kc), dev(vc), out, M, H, Hkv, D, pos, scale)
    got = host(out)
    ref = _oracle_rows(orc, q, kc, vc, H, Hkv, D, pos, np.float32(scale))
    err = normwise_rel_err(got, ref)
    print("prefill attention H=%d/%d D=%d M=%d pos=%d: %.2e" % (H, Hkv, D, M, pos, err))
    assert np.isfinite(got).all() and err <= 1e-5


def test_prefill_attention_errors():
    q = torch.zeros(20, 2048, device="cuda")
    c = torch.zeros(64, 8, 64, device="cuda")
    out = torch.zeros(20, 2048, device="cuda")
    ws = torch.zeros(16, device="cuda")
    with pytest.raises(cri.CretifError):  # workspace too small
        cri.prefill_attention(q, 2048, c, c, out, 20, 32, 8, 64, 0, 0.125, workspace=ws)
    with pytest.raises(cri.CretifError):  # ldq below n_heads * head_dim
        cri.prefill_attention(q, 1024, c, c, out, 20, 32, 8, 64, 0, 0.125)
    with pytest.raises(cri.CretifError):  # head_dim past the layout
        cri.prefill_attention(q, 2048, c, c, out, 20, 8, 8, 256, 0, 0.125)
    with pytest.raises(cri.CretifError):  # misaligned output
        cri.prefill_attention(q, 2048, c, c, out.view(-1)[1:].view(-1)[:20 * 2047].view(20, 2047), 20, 32, 8, 64, 0,
                              0.125)
