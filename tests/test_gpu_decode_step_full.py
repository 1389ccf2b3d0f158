"""GPU parity of the full BASELINE config-5 decode step: all 16 Llama-3.2-1B-shaped layers plus
the Q6_K 128256 x 2048 LM head, the step bench.py times, at M = 1 and M = 16.

Each layer is checked on the GPU's own input to it: cri_decoder_forward_taps writes the residual
stream entering every layer and the final norm, and the oracle's layer (oracle.decode_layer,
ref:src/model.cu:887-1019) run on tap i must give tap i + 1 within 1e-5 normwise (the M <= 16
matmul bar), with the K/V rows it appends within the same bar (k: plus the rotation-angle term of
test_gpu_decode_step.py).  The LM head is checked the same way on the last tap.

End to end (token ids -> logits against oracle.decode_step's 16 layers) the bar is derived, not
chosen: every layer's own error is at most 1e-5 of the stream, and the residual connection carries
each one to the output to first order (a block adds a contribution far smaller than the stream:
RMSNorm-ed inputs, weights ~N(0, 0.02)), so the logits may differ by at most the sum of the
per-layer bars plus the head's: (n_layers + 1) * 1e-5.  The measured errors are printed.

A replay of the captured step equals the eager step bit for bit, and the tapped call gives the
same logits as the untapped one (the taps only read)."""
import numpy as np
import pytest

from conftest import normwise_rel_err

torch = pytest.importorskip("torch")
import cretif_amd as cri  # noqa: E402
from test_gpu_decode_step import LLAMA, from_device, load_cache, make_decoder, make_model, random_cache  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-5
N_LAYERS = 16
MAX_SEQ = 2048


@pytest.fixture(scope="module")
def llama16():
    m = make_model(N_LAYERS, **LLAMA)
    dec = make_decoder(m, max_seq=MAX_SEQ)
    return m, dec


def run_taps(m, dec, ids, pos, kc, vc):
    M = len(ids)
    load_cache(dec, kc, vc)
    dids = torch.from_numpy(np.asarray(ids, np.int32)).cuda()
    logits = torch.full((M, m["vocab"]), float("nan"), device="cuda")
    nxt = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    taps = torch.full((N_LAYERS + 1, M, m["dim"]), float("nan"), device="cuda")
    dec.set_position(pos)
    dec.forward_taps(dids, M, logits, taps, nxt)
    torch.cuda.synchronize()
    return logits.cpu().numpy(), nxt.cpu().numpy(), taps.cpu().numpy()


@pytest.mark.parametrize("M,pos", [(1, 2047), (16, 2032)])
def test_full_step_layer_by_layer(orc, llama16, M, pos):
    m, dec = llama16
    kc, vc = random_cache(m, MAX_SEQ, 4000 + M)
    ids = np.random.default_rng(100 + M).integers(0, m["vocab"], M).astype(np.int32)
    logits, nxt, taps = run_taps(m, dec, ids, pos, kc, vc)
    eps = m["eps"]
    # tap 0: the token rows
    assert np.array_equal(taps[0], orc.embed(m, list(ids)))
    k_tol = TOL + (pos + M) * 2.0 ** -23
    shape = (MAX_SEQ, m["n_kv_heads"], m["head_dim"])
    worst = 0.0
    for i in range(N_LAYERS):
        kci, vci = kc[i].copy(), vc[i].copy()
        _, normed = orc.rmsnorm_residual(taps[i], None, m["layers"][i]["attn_norm"], eps)
        hidden, ffn_out = orc.decode_layer(m, i, taps[i], normed, pos, kci, vci)
        ref = hidden + ffn_out  # the stream entering layer i + 1 (one fp32 add, as the next norm adds it)
        err = normwise_rel_err(taps[i + 1], ref)
        worst = max(worst, err)
        ka, va = dec.kv_cache(i)
        gk, gv = from_device(ka, shape), from_device(va, shape)
        ek = normwise_rel_err(gk[pos:pos + M], kci[pos:pos + M])
        ev = normwise_rel_err(gv[pos:pos + M], vci[pos:pos + M])
        print("M=%d layer %2d: stream err %.2e, k rows %.2e, v rows %.2e" % (M, i, err, ek, ev))
        assert err <= TOL, (i, err)
        assert ek <= k_tol and ev <= TOL, (i, ek, ev)
    # the LM head on the GPU's final stream
    _, normed = orc.rmsnorm_residual(taps[N_LAYERS], None, m["out_norm"], eps)
    head_ref, head_ids = orc.lm_head(m, normed)
    eh = normwise_rel_err(logits, head_ref)
    print("M=%d LM head on the GPU's stream: %.2e (worst layer %.2e)" % (M, eh, worst))
    assert eh <= TOL
    assert np.array_equal(nxt, np.argmax(logits, axis=1))
    # end to end from the token ids
    ref, ref_ids = orc.decode_step(m, list(ids), pos, [k.copy() for k in kc], [v.copy() for v in vc])
    bar = (N_LAYERS + 1) * TOL
    e2e = normwise_rel_err(logits, ref)
    print("M=%d end-to-end logits: %.2e (bar %.1e)" % (M, e2e, bar))
    assert e2e <= bar
    gap_bar = 2 * bar * np.max(np.abs(ref))
    for r in range(M):
        top2 = np.sort(ref[r])[-2:]
        if top2[1] - top2[0] > gap_bar:
            assert nxt[r] == ref_ids[r]


@pytest.mark.parametrize("M,pos", [(1, 2047), (16, 2032)])
def test_full_step_replay_equals_eager_and_taps(llama16, M, pos):
    m, dec = llama16
    kc, vc = random_cache(m, MAX_SEQ, 5000 + M)
    ids = torch.from_numpy((np.arange(M, dtype=np.int32) * 7919 + 11) % m["vocab"]).cuda()
    tapped, _, _ = run_taps(m, dec, ids.cpu().numpy(), pos, kc, vc)
    load_cache(dec, kc, vc)
    a = torch.empty(M, m["vocab"], device="cuda")
    dec.set_position(pos)
    dec.forward(ids, M, a)
    eager = a.cpu().numpy().copy()
    assert np.array_equal(eager.view(np.uint32), tapped.view(np.uint32))
    load_cache(dec, kc, vc)
    s = torch.cuda.Stream()
    b = torch.empty(M, m["vocab"], device="cuda")
    with torch.cuda.stream(s):
        dec.capture(ids, M, b, None, stream=s)
        for _ in range(2):
            dec.set_position(pos, stream=s)
            dec.replay(stream=s)
            s.synchronize()
            assert np.array_equal(b.cpu().numpy().view(np.uint32), eager.view(np.uint32))
    torch.cuda.synchronize()


def test_step_weight_bytes_counts_token_rows(llama16):
    m, dec = llama16
    layers = sum(m["layers"][i][k][1].nbytes for i in range(N_LAYERS)
                 for k in ("q", "k", "v", "o", "gate", "up", "down"))
    norms = (2 * N_LAYERS + 1) * m["dim"] * 4
    tok_row = m["tok"][1].nbytes // m["vocab"]
    for M in (1, 16):
        assert dec.step_weight_bytes(M) == layers + norms + m["lm"][1].nbytes + M * tok_row
    assert dec.weight_bytes == layers + norms + m["lm"][1].nbytes + m["tok"][1].nbytes
