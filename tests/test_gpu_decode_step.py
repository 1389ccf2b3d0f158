"""GPU parity of the decode step (cri_decoder_*, C++ cuinfer::DecodeStep): the
BASELINE config-5 step at Llama-3.2-1B shapes -- Q4_K q/k/v/o/gate/up/down
(2048x2048, 512x2048, 8192x2048, 2048x8192), a Q6_K 128256x2048 LM head, an fp32
KV cache of 2048 positions ~ N(0, 1), 32 query heads over 8 KV heads -- with the
values chained through the layers, against the oracle's composition of the
reference's forward pass (oracle.decode_step: orc_rmsnorm_residual, the
reference's dequant + sequential matmul, orc_rope, orc_decode_attention per
causal row, orc_silu_mul, orc_argmax; ref:src/model.cu:876-1039).

Two full-size layers are run (the oracle composes 16 in about 8x the CPU time;
every layer is the same code).  Weights are random valid blocks
(quant.random_blocks: std ~0.02) so that the host can make 2 x 61M weights in
seconds; both sides read the same bytes.

Bars (normwise, ||x - ref||_inf / ||ref||_inf): logits and the appended KV rows
<= 1e-5 for batches of up to 16 tokens (the fp32-accurate matmul bar; the step
chains 2 layers of them); 2e-3 for a 17-token batch, which runs the prefill GEMM
on fp16 operands (its stated bar is 1e-3 per product).  Greedy ids: the GPU's
argmax of its own logits exactly, and the oracle's wherever the oracle's top two
logits are further apart than the logits' error bound.  A replayed graph equals
the eager step bit for bit (the M <= 16 kernels are deterministic)."""
import ctypes

import numpy as np
import pytest

from conftest import normwise_rel_err

torch = pytest.importorskip("torch")
import cretif_amd as cri  # noqa: E402
from cretif_amd import quant  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-5
PREFILL_TOL = 2e-3
LLAMA = dict(dim=2048, n_heads=32, n_kv_heads=8, head_dim=64, ffn=8192, vocab=128256)


def _hip():
    path = next(ln.split()[-1] for ln in open("/proc/self/maps") if "libamdhip64" in ln)
    h = ctypes.CDLL(path)
    h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return h


def to_device(addr, a):
    a = np.ascontiguousarray(a, np.float32)
    torch.cuda.synchronize()
    assert _hip().hipMemcpy(addr, a.ctypes.data, a.nbytes, 1) == 0  # hipMemcpyHostToDevice


def from_device(addr, shape):
    out = np.empty(shape, np.float32)
    torch.cuda.synchronize()
    assert _hip().hipMemcpy(out.ctypes.data, addr, out.nbytes, 2) == 0  # hipMemcpyDeviceToHost
    return out


def tiled(fmt, N, K, seed, rows=4096):
    """N rows from `rows` random rows repeated (the large tables; the row pattern still
    differs from one tile to the next in position)."""
    base = quant.random_blocks(fmt, rows, K, seed).reshape(rows, -1)
    return np.ascontiguousarray(np.tile(base, (-(-N // rows), 1))[:N]).ravel()


def make_model(n_layers, dim, n_heads, n_kv_heads, head_dim, ffn, vocab, seed=1100, fmts=None, tok="q8_0",
               lm="q6_k", big_tables=True):
    fmts = fmts or {}
    rng = np.random.default_rng(seed)
    layers = []
    for i in range(n_layers):
        b = seed + 10 * i

        def w(name, n, k, s):
            f = fmts.get(name, "q4_k")
            return f, quant.random_blocks(f, n, k, b + s)

        layers.append({
            "attn_norm": (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32),
            "ffn_norm": (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32),
            "q": w("q", n_heads * head_dim, dim, 0), "k": w("k", n_kv_heads * head_dim, dim, 1),
            "v": w("v", n_kv_heads * head_dim, dim, 2), "o": w("o", dim, n_heads * head_dim, 3),
            "gate": w("gate", ffn, dim, 4), "up": w("up", ffn, dim, 5), "down": w("down", dim, ffn, 6)})
    make = tiled if big_tables else (lambda f, n, k, s: quant.random_blocks(f, n, k, s))
    if tok == "fp32":
        table = (rng.standard_normal(vocab * dim) * 0.02).astype(np.float32)
    else:
        table = make(tok, vocab, dim, seed + 500)
    return {"n_heads": n_heads, "n_kv_heads": n_kv_heads, "head_dim": head_dim, "dim": dim, "ffn": ffn,
            "vocab": vocab, "eps": 1e-5, "theta": 500000.0, "tok": (tok, table), "layers": layers,
            "out_norm": (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32),
            "lm": None if lm is None else (lm, make(lm, vocab, dim, seed + 501))}


def make_decoder(m, max_seq, max_batch=16):
    d = cri.Decoder(len(m["layers"]), m["dim"], m["n_heads"], m["n_kv_heads"], m["head_dim"], m["ffn"], m["vocab"],
                    max_seq, max_batch=max_batch, rms_norm_eps=m["eps"], rope_theta=m["theta"])
    for i, L in enumerate(m["layers"]):
        d.set_layer(i, L["attn_norm"], L["ffn_norm"], **{k: L[k] for k in ("q", "k", "v", "o", "gate", "up", "down")})
    d.set_embedding(*m["tok"])
    d.set_output(m["out_norm"], m["lm"])
    return d


def random_cache(m, T, seed):
    rng = np.random.default_rng(seed)
    shape = (T, m["n_kv_heads"], m["head_dim"])
    return ([rng.standard_normal(shape).astype(np.float32) for _ in m["layers"]],
            [rng.standard_normal(shape).astype(np.float32) for _ in m["layers"]])


def load_cache(dec, kc, vc):
    for i, (k, v) in enumerate(zip(kc, vc)):
        ka, va = dec.kv_cache(i)
        to_device(ka, k)
        to_device(va, v)


def check_ids(got_ids, logits, ref_logits, ref_ids, tol):
    # the GPU's ids are the argmax (first index of the maximum) of its own logits
    assert np.array_equal(got_ids, np.argmax(logits, axis=1))
    bound = 2 * tol * np.max(np.abs(ref_logits))
    for r in range(ref_logits.shape[0]):
        top2 = np.sort(ref_logits[r])[-2:]
        if top2[1] - top2[0] > bound:
            assert got_ids[r] == ref_ids[r]


@pytest.fixture(scope="module")
def llama2():
    """Two full-size Llama-3.2-1B layers, Q6_K LM head, Q8_0 token table; cache of 2048."""
    m = make_model(2, **LLAMA)
    dec = make_decoder(m, max_seq=2048)
    return m, dec


@pytest.mark.parametrize("M,pos", [(1, 2047), (16, 2032), (1, 0), (5, 700), (8, 2040), (2, 1500)])
def test_step_llama_shapes(orc, llama2, M, pos):
    m, dec = llama2
    kc, vc = random_cache(m, 2048, 3000 + pos)
    load_cache(dec, kc, vc)
    ids = np.random.default_rng(M + pos).integers(0, m["vocab"], M).astype(np.int32)
    dids = torch.from_numpy(ids).cuda()
    logits = torch.full((M, m["vocab"]), float("nan"), device="cuda")
    nxt = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    dec.set_position(pos)
    dec.forward(dids, M, logits, nxt)
    assert dec.position == pos + M
    got = logits.cpu().numpy()
    ref, ref_ids = orc.decode_step(m, list(ids), pos, kc, vc)
    err = normwise_rel_err(got, ref)
    print("decode step M=%d pos=%d: logits normwise err %.2e" % (M, pos, err))
    assert err <= TOL
    check_ids(nxt.cpu().numpy(), got, ref, ref_ids, TOL)
    # the rows appended to every layer's cache: rotated k and plain v.  The rotation angle
    # pos * freq turns a one-ulp difference in the frequency (fp32 powf here and there) into
    # pos ulps of the angle, so the k bar adds (pos + M) * 2^-23 to the matmul bar
    k_tol = TOL + (pos + M) * 2.0 ** -23
    for i in range(len(m["layers"])):
        ka, va = dec.kv_cache(i)
        shape = (2048, m["n_kv_heads"], m["head_dim"])
        gk, gv = from_device(ka, shape), from_device(va, shape)
        assert normwise_rel_err(gk[pos:pos + M], kc[i][pos:pos + M]) <= k_tol
        assert normwise_rel_err(gv[pos:pos + M], vc[i][pos:pos + M]) <= TOL
        assert np.array_equal(gk[:pos], kc[i][:pos]) and np.array_equal(gk[pos + M:], kc[i][pos + M:])


def test_graph_replay_equals_eager_and_generates(orc, llama2):
    m, dec = llama2
    kc, vc = random_cache(m, 2048, 77)
    load_cache(dec, kc, vc)
    pos0, steps = 1000, 4
    s = torch.cuda.Stream()
    ids = torch.tensor([123], dtype=torch.int32, device="cuda")
    logits = torch.empty(1, m["vocab"], device="cuda")
    # eager greedy loop
    eager_ids, eager_logits = [], []
    dec.set_position(pos0)
    cur = ids.clone()
    for _ in range(steps):
        nxt = torch.empty(1, dtype=torch.int32, device="cuda")
        dec.forward(cur, 1, logits, nxt)
        eager_logits.append(logits.cpu().numpy().copy())
        eager_ids.append(int(nxt.cpu()[0]))
        cur = nxt
    # the same loop as replays of one captured step whose next_ids is its token_ids
    load_cache(dec, kc, vc)
    buf = ids.clone()
    with torch.cuda.stream(s):
        dec.capture(buf, 1, logits, buf, stream=s)
        dec.set_position(pos0, stream=s)
        for t in range(steps):
            dec.replay(stream=s)
            s.synchronize()
            assert np.array_equal(logits.cpu().numpy().view(np.uint32), eager_logits[t].view(np.uint32))
            assert int(buf.cpu()[0]) == eager_ids[t]
    assert dec.position == pos0 + steps
    # and the first step against the oracle
    ref, ref_ids = orc.decode_step(m, [123], pos0, *random_cache(m, 2048, 77))
    assert normwise_rel_err(eager_logits[0], ref) <= TOL


def test_batch16_replay_equals_eager(llama2):
    m, dec = llama2
    kc, vc = random_cache(m, 2048, 5)
    load_cache(dec, kc, vc)
    M, pos = 16, 100
    ids = torch.from_numpy(np.arange(M, dtype=np.int32) * 7919).cuda()
    a = torch.empty(M, m["vocab"], device="cuda")
    dec.set_position(pos)
    dec.forward(ids, M, a)
    eager = a.cpu().numpy().copy()
    load_cache(dec, kc, vc)
    s = torch.cuda.Stream()
    b = torch.empty(M, m["vocab"], device="cuda")
    with torch.cuda.stream(s):
        dec.capture(ids, M, b, None, stream=s)
        dec.set_position(pos, stream=s)
        dec.replay(stream=s)
    s.synchronize()
    assert np.array_equal(b.cpu().numpy().view(np.uint32), eager.view(np.uint32))


@pytest.mark.parametrize("M", [17, 12, 3, 1])
def test_step_mixed_formats_tied_fp32_head(orc, M):
    # q/k/v and gate/up of different formats (three / two separate matrices), an FP32 token
    # table tied to the LM head (matmul_transposed_b), head_dim 128 (the 8-slice attention
    # layout); for M = 3 and 12 every format's K split over workgroups with the step's workspace
    # (the RMSNorm prologue included), for M = 17 the unfused path (rmsnorm_residual, prefill GEMM,
    # silu_mul), for M = 1 the first layer's down projection split into partial sums that the
    # separate q, k and v GEMVs of the second add up (the FP32 head takes a whole residual)
    m = make_model(2, dim=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=1024, vocab=1000, seed=7,
                   fmts={"q": "q8_0", "k": "q4_0", "v": "q5_0", "o": "fp16", "gate": "q6_k", "up": "q4_k",
                         "down": "q8_0"}, tok="fp32", lm=None, big_tables=False)
    dec = make_decoder(m, max_seq=256, max_batch=32)
    kc, vc = random_cache(m, 256, 9)
    load_cache(dec, kc, vc)
    pos = 40
    ids = np.random.default_rng(M).integers(0, m["vocab"], M).astype(np.int32)
    logits = torch.empty(M, m["vocab"], device="cuda")
    nxt = torch.empty(M, dtype=torch.int32, device="cuda")
    dec.set_position(pos)
    dec.forward(torch.from_numpy(ids).cuda(), M, logits, nxt)
    got = logits.cpu().numpy()
    ref, ref_ids = orc.decode_step(m, list(ids), pos, kc, vc)
    tol = PREFILL_TOL if M > 16 else TOL
    err = normwise_rel_err(got, ref)
    print("mixed-format step M=%d: normwise err %.2e" % (M, err))
    assert err <= tol
    check_ids(nxt.cpu().numpy(), got, ref, ref_ids, tol)


@pytest.mark.parametrize("fmt,M", [("q8_0", 12), ("q6_k", 9), ("fp16", 16), ("q5_0", 1), ("q6_k", 1),
                                   ("q4_k", 2), ("q8_0", 5), ("q4_0", 8), ("q6_k", 4), ("fp16", 3)])
def test_step_fused_projections_split(orc, fmt, M):
    # one format throughout, so q/k/v and gate/up are stored fused; at 2..16 rows their K is
    # split over workgroups and the partial sums are left for RoPE (q/k/v) and for the down
    # projection's prologue (a two-way gate/up split) to add up; at one row the q/k/v GEMV
    # rotates and appends to the caches in its epilogue
    m = make_model(2, dim=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=2048, vocab=3000, seed=17,
                   fmts={n: fmt for n in ("q", "k", "v", "o", "gate", "up", "down")}, tok="q8_0", lm=fmt,
                   big_tables=False)
    dec = make_decoder(m, max_seq=512)
    kc, vc = random_cache(m, 512, 21)
    load_cache(dec, kc, vc)
    pos = 300
    ids = np.random.default_rng(M + 5).integers(0, m["vocab"], M).astype(np.int32)
    logits = torch.empty(M, m["vocab"], device="cuda")
    nxt = torch.empty(M, dtype=torch.int32, device="cuda")
    dec.set_position(pos)
    dec.forward(torch.from_numpy(ids).cuda(), M, logits, nxt)
    got = logits.cpu().numpy()
    ref, ref_ids = orc.decode_step(m, list(ids), pos, kc, vc)
    err = normwise_rel_err(got, ref)
    print("fused-projection step %s M=%d: normwise err %.2e" % (fmt, M, err))
    assert err <= TOL
    check_ids(nxt.cpu().numpy(), got, ref, ref_ids, TOL)
    k_tol = TOL + (pos + M) * 2.0 ** -23
    for i in range(len(m["layers"])):
        ka, va = dec.kv_cache(i)
        shape = (512, m["n_kv_heads"], m["head_dim"])
        gk, gv = from_device(ka, shape), from_device(va, shape)
        assert normwise_rel_err(gk[pos:pos + M], kc[i][pos:pos + M]) <= k_tol
        assert normwise_rel_err(gv[pos:pos + M], vc[i][pos:pos + M]) <= TOL


@pytest.mark.parametrize("M,pos,max_seq", [(16, 3000, 4096), (8, 5000, 8192), (5, 8180, 8192)])
def test_step_long_context(orc, M, pos, max_seq):
    # past 64 x 32 positions the multi-row attention's chunks hold two (4096) or three or more
    # (8192) 32-position tiles each
    m = make_model(1, dim=256, n_heads=8, n_kv_heads=2, head_dim=64, ffn=512, vocab=500, seed=23,
                   big_tables=False)
    dec = make_decoder(m, max_seq=max_seq)
    kc, vc = random_cache(m, max_seq, 31)
    load_cache(dec, kc, vc)
    ids = np.random.default_rng(pos).integers(0, m["vocab"], M).astype(np.int32)
    logits = torch.empty(M, m["vocab"], device="cuda")
    dec.set_position(pos)
    dec.forward(torch.from_numpy(ids).cuda(), M, logits)
    ref, _ = orc.decode_step(m, list(ids), pos, kc, vc)
    err = normwise_rel_err(logits.cpu().numpy(), ref)
    print("long-context step M=%d pos=%d: normwise err %.2e" % (M, pos, err))
    assert err <= TOL


def test_decoder_errors():
    m = make_model(1, dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=100, big_tables=False)
    with pytest.raises(cri.CretifError):  # n_heads not a multiple of n_kv_heads
        cri.Decoder(1, 256, 4, 3, 64, 512, 100, 64)
    with pytest.raises(cri.CretifError):  # head_dim past the attention layout
        cri.Decoder(1, 256, 1, 1, 256, 512, 100, 64)
    d = cri.Decoder(1, 256, 4, 2, 64, 512, 100, 8, max_batch=4)
    ids = torch.zeros(8, dtype=torch.int32, device="cuda")
    out = torch.empty(8, 100, device="cuda")
    with pytest.raises(cri.CretifError):  # no weights yet
        d.forward(ids, 1, out)
    L = m["layers"][0]
    d.set_layer(0, L["attn_norm"], L["ffn_norm"], **{k: L[k] for k in ("q", "k", "v", "o", "gate", "up", "down")})
    d.set_embedding(*m["tok"])
    d.set_output(m["out_norm"], m["lm"])
    with pytest.raises(cri.CretifError):  # M above max_batch
        d.forward(ids, 5, out)
    d.forward(ids, 4, out)
    d.forward(ids, 4, out)
    assert d.position == 8
    with pytest.raises(cri.CretifError) as e:  # past max_seq_len
        d.forward(ids, 1, out)
    assert e.value.status == -2
    with pytest.raises(cri.CretifError):
        d.replay()  # nothing captured
    with pytest.raises(cri.CretifError):
        d.set_position(9)
    d.set_position(0)
    torch.cuda.synchronize()


def test_setters_drop_the_captured_graph_and_keep_old_weights_on_failure():
    # every setter discards a captured graph (it holds the old buffers and kernel choices), and a
    # set_layer that fails part way (a null matrix after the others were copied) leaves the old
    # layer in place: the next step gives the same logits bit for bit
    m = make_model(2, dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=300, seed=41,
                   big_tables=False)
    dec = make_decoder(m, max_seq=64)
    kc, vc = random_cache(m, 64, 42)
    ids = torch.tensor([5, 17], dtype=torch.int32, device="cuda")
    a = torch.empty(2, m["vocab"], device="cuda")
    load_cache(dec, kc, vc)
    dec.set_position(10)
    dec.forward(ids, 2, a)
    before = a.cpu().numpy().copy()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        dec.capture(ids, 2, a, None, stream=s)
        dec.set_position(10, stream=s)
        dec.replay(stream=s)
    s.synchronize()
    L = m["layers"][1]
    mats = {k: L[k] for k in ("q", "k", "v", "o", "gate", "up", "down")}
    dec.set_layer(1, L["attn_norm"], L["ffn_norm"], **mats)
    with pytest.raises(cri.CretifError):
        dec.replay()  # discarded by set_layer
    with pytest.raises(cri.CretifError):
        dec.set_layer(1, L["attn_norm"], L["ffn_norm"], **dict(mats, down=(mats["down"][0], None)))
    for setter in (lambda: dec.set_embedding(*m["tok"]), lambda: dec.set_output(m["out_norm"], m["lm"])):
        with torch.cuda.stream(s):
            dec.capture(ids, 2, a, None, stream=s)
        setter()
        with pytest.raises(cri.CretifError):
            dec.replay()
    load_cache(dec, kc, vc)
    dec.set_position(10)
    dec.forward(ids, 2, a)
    assert np.array_equal(a.cpu().numpy().view(np.uint32), before.view(np.uint32))


@pytest.mark.parametrize("dim,M", [(4096, 1), (5120, 4), (5120, 12), (4352, 1), (4352, 3)])
def test_step_wide_models(orc, dim, M):
    # branches the Llama-3.2-1B shapes do not reach: a 4096-wide model at one token (the fused
    # q/k/v GEMV with RoPE on the K-sliced kernel), widths past 4096 at 2..16 tokens (the q/k/v
    # partial sums added up by RoPE, the two-way gate/up SwiGLU on the skinny kernel's own sums
    # of squares), and a width the K-sliced and 32-lane RoPE GEMVs decline (4352 = 17 x 256) at
    # one token (the RMSNorm GEMV, then the RoPE kernel) and at three
    m = make_model(1, dim=dim, n_heads=dim // 64, n_kv_heads=4, head_dim=64, ffn=2 * dim, vocab=700, seed=dim + M,
                   big_tables=False)
    dec = make_decoder(m, max_seq=128)
    kc, vc = random_cache(m, 128, dim)
    load_cache(dec, kc, vc)
    pos = 50
    ids = np.random.default_rng(dim + M).integers(0, m["vocab"], M).astype(np.int32)
    logits = torch.empty(M, m["vocab"], device="cuda")
    dec.set_position(pos)
    dec.forward(torch.from_numpy(ids).cuda(), M, logits)
    ref, _ = orc.decode_step(m, list(ids), pos, kc, vc)
    err = normwise_rel_err(logits.cpu().numpy(), ref)
    print("wide-model step dim=%d M=%d: normwise err %.2e" % (dim, M, err))
    assert err <= TOL


@pytest.mark.parametrize("pos", [0, 1000])
def test_prompt_two_layers_through_gqa(orc, pos):
    # a 512-token prompt through two full-size Llama-3.2-1B layers: above 16 rows the step runs the
    # reference's prefill flow (ref:src/attention.cu:809-871), Q K^T and P V on batched_matmul_gqa
    # around a causal softmax (pinned on its own at 1e-5 in test_gpu_attention.py), with every
    # projection on the prefill GEMMs (fp16 operands; the stated bar 2e-3).  FP16 weights ~N(0, 0.02):
    # the random-block Q4_K weights of the other tests are not zero-mean (d sc q - dmin mn is mostly
    # positive), which gives q and k a large shared component, sharp attention rows, and a softmax
    # that amplifies the fp16 operand rounding past the bar (~6e-2 at 512 tokens, the same with the
    # multi-row attention kernel that served prompts before)
    m = make_model(2, dim=2048, n_heads=32, n_kv_heads=8, head_dim=64, ffn=8192, vocab=2000, seed=61 + pos,
                   fmts={n: "fp16" for n in ("q", "k", "v", "o", "gate", "up", "down")}, tok="q8_0", lm="fp16",
                   big_tables=False)
    dec = make_decoder(m, max_seq=2048, max_batch=512)
    kc, vc = random_cache(m, 2048, 62 + pos)
    load_cache(dec, kc, vc)
    M = 512
    ids = np.random.default_rng(pos + 3).integers(0, m["vocab"], M).astype(np.int32)
    logits = torch.empty(M, m["vocab"], device="cuda")
    dec.set_position(pos)
    dec.forward(torch.from_numpy(ids).cuda(), M, logits)
    got = logits.cpu().numpy()
    ref, _ = orc.decode_step(m, list(ids), pos, kc, vc)
    err = normwise_rel_err(got, ref)
    print("prompt M=%d pos=%d: logits normwise err %.2e" % (M, pos, err))
    assert err <= PREFILL_TOL
    for i in range(2):
        ka, va = dec.kv_cache(i)
        shape = (2048, m["n_kv_heads"], m["head_dim"])
        gk, gv = from_device(ka, shape), from_device(va, shape)
        assert normwise_rel_err(gk[pos:pos + M], kc[i][pos:pos + M]) <= PREFILL_TOL + (pos + M) * 2.0 ** -23
        assert normwise_rel_err(gv[pos:pos + M], vc[i][pos:pos + M]) <= PREFILL_TOL


@pytest.mark.parametrize("M,pos", [(512, 0), (17, 100), (12, 40), (5, 700), (1, 9)])
def test_prefill_last_row_equals_forward(orc, M, pos):
    # cri_decoder_prefill (generate()'s use of a prompt, ref:src/model.cu:1063-1078): forward()'s
    # layers on the M tokens, then the final RMSNorm, LM head and argmax of the last token only.
    # The caches and position must match a forward() of the same tokens bit for bit (the prefill
    # GEMMs' K splits add their partial sums in a fixed order through the step's workspace), its
    # logits forward()'s last row (above 16 rows those come from the fp16-operand prefill GEMM:
    # the 2e-3 bar) and, up to 17 rows, the oracle's last row; next_id is the argmax of its own
    # logits.  M = 1 is forward().
    big = M > 16
    fm = {n: "fp16" for n in ("q", "k", "v", "o", "gate", "up", "down")} if big else None
    m = make_model(2, dim=2048, n_heads=32, n_kv_heads=8, head_dim=64, ffn=8192, vocab=2000, seed=71 + M,
                   fmts=fm, tok="q8_0", lm="fp16" if big else "q6_k", big_tables=False)
    dec = make_decoder(m, max_seq=2048, max_batch=max(M, 16))
    kc, vc = random_cache(m, 2048, 72 + M)
    ids = np.random.default_rng(M + pos).integers(0, m["vocab"], M).astype(np.int32)
    dids = torch.from_numpy(ids).cuda()
    V, shape = m["vocab"], (2048, m["n_kv_heads"], m["head_dim"])

    load_cache(dec, kc, vc)
    dec.set_position(pos)
    full = torch.full((M, V), float("nan"), device="cuda")
    dec.forward(dids, M, full)
    caches = [tuple(from_device(a, shape) for a in dec.kv_cache(i)) for i in range(2)]

    load_cache(dec, kc, vc)
    dec.set_position(pos)
    last = torch.full((V,), float("nan"), device="cuda")
    nid = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    dec.prefill(dids, M, last, nid)
    assert dec.position == pos + M
    got = last.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert int(nid.cpu().numpy()[0]) == int(np.argmax(got))
    tol = PREFILL_TOL if big else TOL
    err = normwise_rel_err(got, full.cpu().numpy()[M - 1])
    print("prefill M=%d pos=%d: last-row logits against forward %.2e" % (M, pos, err))
    assert err <= tol
    for i in range(2):
        gk, gv = (from_device(a, shape) for a in dec.kv_cache(i))
        assert np.array_equal(gk, caches[i][0]) and np.array_equal(gv, caches[i][1])
    if M <= 17:
        ref, _ = orc.decode_step(m, list(ids), pos, kc, vc)
        assert normwise_rel_err(got, ref[M - 1]) <= tol


@pytest.mark.parametrize("M,pos", [(16, 0), (4, 0), (8, 31), (16, 120), (5, 1000), (16, 1008)])
def test_batch_attention_rope_nan_cache(orc, M, pos):
    # 4..16 rows on the multi-row attention: every cache row from pos on holds NaN before the step,
    # so a product that read a row before the step wrote it, or one past the batch's last position
    # (a clamped read past a chunk's end, the V operand's 0 * NaN), would poison the logits.
    # Positions: 0 (every row the batch's own), new rows across a tile boundary (31) and across a
    # chunk boundary (120 at 16 rows: chunks of one tile), the last positions of the cache (1008 + 16
    # = 1024).  Rows past the batch stay NaN; a replay equals the eager step.
    m = make_model(2, dim=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=1024, vocab=900, seed=81 + pos,
                   big_tables=False)
    max_seq = 1024
    dec = make_decoder(m, max_seq=max_seq)
    kc, vc = random_cache(m, max_seq, 82 + pos)
    for arr in kc + vc:
        arr[pos:] = np.nan
    load_cache(dec, kc, vc)
    ids = np.random.default_rng(83 + M).integers(0, m["vocab"], M).astype(np.int32)
    dids = torch.from_numpy(ids).cuda()
    a = torch.empty(M, m["vocab"], device="cuda")
    dec.set_position(pos)
    dec.forward(dids, M, a)
    eager = a.cpu().numpy().copy()
    rk, rv = [k.copy() for k in kc], [v.copy() for v in vc]
    ref, _ = orc.decode_step(m, list(ids), pos, rk, rv)
    err = normwise_rel_err(eager, ref)
    print("batch M=%d pos=%d, NaN from pos on: normwise err %.2e" % (M, pos, err))
    assert np.isfinite(eager).all() and err <= TOL
    k_tol = TOL + (pos + M) * 2.0 ** -23
    for i in range(len(m["layers"])):
        ka, va = dec.kv_cache(i)
        shape = (max_seq, m["n_kv_heads"], m["head_dim"])
        gk, gv = from_device(ka, shape), from_device(va, shape)
        assert normwise_rel_err(gk[pos:pos + M], rk[i][pos:pos + M]) <= k_tol
        assert normwise_rel_err(gv[pos:pos + M], rv[i][pos:pos + M]) <= TOL
        assert np.array_equal(gk[:pos], kc[i][:pos]) and np.isnan(gk[pos + M:]).all()
    # a captured step replayed at the same position on the same cache: the same bits
    load_cache(dec, kc, vc)
    s = torch.cuda.Stream()
    b = torch.empty(M, m["vocab"], device="cuda")
    with torch.cuda.stream(s):
        dec.set_position(pos, stream=s)
        dec.capture(dids, M, b, None, stream=s)
        dec.set_position(pos, stream=s)
        dec.replay(stream=s)
    s.synchronize()
    assert np.array_equal(b.cpu().numpy(), eager)


@pytest.mark.parametrize("head_dim", [64, 128])
def test_prompt_row_blocks_nan_cache_and_replay(orc, head_dim):
    # 600 rows: at head_dim 64 the multi-row split attention takes them at once, otherwise the
    # reference's flow on batched_matmul_gqa in two row blocks (512 + 88); cache rows past the
    # step's positions hold NaN, which no product may read; a graph captured at one position (its
    # products span the whole cache) and replayed at another equals the eager step there
    m = make_model(2, dim=512, n_heads=512 // head_dim, n_kv_heads=2, head_dim=head_dim, ffn=1024, vocab=900, seed=71,
                   fmts={n: "fp16" for n in ("q", "k", "v", "o", "gate", "up", "down")}, tok="q8_0", lm="fp16",
                   big_tables=False)
    max_seq = 1024
    dec = make_decoder(m, max_seq=max_seq, max_batch=640)
    kc, vc = random_cache(m, max_seq, 72)
    M, pos = 600, 37
    for arr in kc + vc:
        arr[pos + M:] = np.nan
    load_cache(dec, kc, vc)
    ids = torch.from_numpy(np.random.default_rng(73).integers(0, m["vocab"], M).astype(np.int32)).cuda()
    a = torch.empty(M, m["vocab"], device="cuda")
    dec.set_position(pos)
    dec.forward(ids, M, a)
    eager = a.cpu().numpy().copy()
    ref, _ = orc.decode_step(m, list(ids.cpu().numpy()), pos, [k.copy() for k in kc], [v.copy() for v in vc])
    err = normwise_rel_err(eager, ref)
    print("prompt M=600 (head_dim %d), NaN past the step: normwise err %.2e" % (head_dim, err))
    assert np.isfinite(eager).all() and err <= PREFILL_TOL
    # captured at another position, replayed at pos: the same logits (the products span the whole
    # cache there, with the extra columns masked and the extra rows zero)
    load_cache(dec, kc, vc)
    s = torch.cuda.Stream()
    b = torch.empty(M, m["vocab"], device="cuda")
    with torch.cuda.stream(s):
        dec.set_position(200, stream=s)
        dec.capture(ids, M, b, None, stream=s)
        dec.set_position(pos, stream=s)
        dec.replay(stream=s)
    s.synchronize()
    assert normwise_rel_err(b.cpu().numpy(), eager) <= 1e-5


@pytest.mark.parametrize("ffn", [1056, 1024])
def test_prompt_swiglu_partial_tile(orc, ffn):
    # the fused gate/up + SiLU * up launch covers 128 output columns per tile: an FFN width that is
    # not a multiple of 128 (1056: the last tile holds 32 columns) and one that is, against the oracle
    m = make_model(2, dim=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=ffn, vocab=700, seed=95 + ffn,
                   fmts={n: "fp16" for n in ("q", "k", "v", "o", "gate", "up", "down")}, tok="q8_0", lm="fp16",
                   big_tables=False)
    M, pos, max_seq = 80, 9, 256
    dec = make_decoder(m, max_seq=max_seq, max_batch=M)
    kc, vc = random_cache(m, max_seq, 96)
    load_cache(dec, kc, vc)
    ids = torch.from_numpy(np.random.default_rng(97).integers(0, m["vocab"], M).astype(np.int32)).cuda()
    a = torch.empty(M, m["vocab"], device="cuda")
    dec.set_position(pos)
    dec.forward(ids, M, a)
    ref, _ = orc.decode_step(m, list(ids.cpu().numpy()), pos, [k.copy() for k in kc], [v.copy() for v in vc])
    err = normwise_rel_err(a.cpu().numpy(), ref)
    print("prompt M=%d ffn=%d: normwise err %.2e" % (M, ffn, err))
    assert err <= PREFILL_TOL


def test_prompt_swiglu_flagged_rows(orc):
    # a prompt's stacked gate/up matrix runs as one launch with SiLU(gate) * up in its epilogue; rows
    # whose activations leave fp16's range (an FFN norm weight of 1e5 makes every row's reach ~1e5)
    # are recomputed there in fp32, both sums and then SiLU * up, as the separate products and the
    # elementwise kernel would; the logits against the oracle at the prefill bar
    m = make_model(2, dim=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=1024, vocab=900, seed=91,
                   fmts={n: "fp16" for n in ("q", "k", "v", "o", "gate", "up", "down")}, tok="q8_0", lm="fp16",
                   big_tables=False)
    m["layers"][0]["ffn_norm"] = (m["layers"][0]["ffn_norm"] * 1e5).astype(np.float32)
    M, pos, max_seq = 64, 5, 256
    dec = make_decoder(m, max_seq=max_seq, max_batch=M)
    kc, vc = random_cache(m, max_seq, 92)
    load_cache(dec, kc, vc)
    ids = torch.from_numpy(np.random.default_rng(93).integers(0, m["vocab"], M).astype(np.int32)).cuda()
    a = torch.empty(M, m["vocab"], device="cuda")
    dec.set_position(pos)
    dec.forward(ids, M, a)
    got = a.cpu().numpy()
    ref, _ = orc.decode_step(m, list(ids.cpu().numpy()), pos, [k.copy() for k in kc], [v.copy() for v in vc])
    err = normwise_rel_err(got, ref)
    print("prompt M=%d, FFN activations ~1e5: normwise err %.2e" % (M, err))
    assert np.isfinite(got).all() and err <= PREFILL_TOL
