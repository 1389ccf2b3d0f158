"""The oracle's decode-step composition (oracle.decode_step) pinned by an independent float64
forward of the reference's quantized forward pass, written here in numpy from
ref:src/model.cu:876-1039 and the kernels it calls -- rmsnorm / rmsnorm_residual
(ref:src/kernels/elementwise.cu:463-504: v = x + r, normed = v * w / sqrt(mean(v^2) + eps)),
rope (ref:src/kernels/elementwise.cu:232-257: pairs (2i, 2i + 1) of each head rotated by
pos / theta^(2i / head_dim)), silu (ref:src/kernels/elementwise.cu:93-99), the fused decode
attention (ref:src/attention.cu:410-494; row t of a batch sees positions <= pos + t,
ref:src/attention.cu:60-75) and the GQA head mapping h -> h / (n_heads / n_kv_heads).  Nothing
here calls oracle/__init__.py except the function under test and, for the planted mistakes,
its building blocks.

The weights are FP16 (exactly representable in float64, so the forward needs no dequantizer),
the token table FP32.  Bar, derived: every fp32 step of the oracle (a matmul over K <= 128
terms, a norm, a softmax over <= 40 positions) is within gamma_K = K 2^-24 ~ 8e-6 relative of
its float64 value; a layer chains ~10 of them and 3 layers plus the head chain ~35, so the
logits are within 35 * 8e-6 ~ 3e-4 normwise.  A composition mistake (the next layer's norm
weight taken from the same layer, the first standalone RMSNorm dropped, the attention output
added to the wrong stream) changes the logits by O(10%), and the planted-mistake cases check
that each one fails the same bar."""
import numpy as np
import pytest

from conftest import normwise_rel_err

BAR = 3e-4
CFG = dict(n_layers=3, dim=64, n_heads=4, n_kv_heads=2, head_dim=16, ffn=128, vocab=50, eps=1e-5, theta=10000.0)


def make_model(seed, tied=False):
    rng = np.random.default_rng(seed)
    c = CFG
    D, F, H, Hkv, hd = c["dim"], c["ffn"], c["n_heads"], c["n_kv_heads"], c["head_dim"]

    def w16(n, k):
        return (rng.standard_normal((n, k)) * 0.15).astype(np.float16)

    layers = []
    for _ in range(c["n_layers"]):
        layers.append({"attn_norm": (1 + 0.2 * rng.standard_normal(D)).astype(np.float32),
                       "ffn_norm": (1 + 0.2 * rng.standard_normal(D)).astype(np.float32),
                       "q": w16(H * hd, D), "k": w16(Hkv * hd, D), "v": w16(Hkv * hd, D), "o": w16(D, H * hd),
                       "gate": w16(F, D), "up": w16(F, D), "down": w16(D, F)})
    table = rng.standard_normal((c["vocab"], D)).astype(np.float32)
    out_norm = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    lm = None if tied else w16(c["vocab"], D)
    # the oracle's model dict: weights as (fmt, bytes)
    om = {"n_heads": H, "n_kv_heads": Hkv, "head_dim": hd, "dim": D, "ffn": F, "vocab": c["vocab"], "eps": c["eps"],
          "theta": c["theta"], "tok": ("fp32", table), "out_norm": out_norm,
          "lm": None if lm is None else ("fp16", lm.view(np.uint8).ravel()),
          "layers": [{"attn_norm": L["attn_norm"], "ffn_norm": L["ffn_norm"],
                      **{k: ("fp16", L[k].view(np.uint8).ravel()) for k in ("q", "k", "v", "o", "gate", "up", "down")}}
                     for L in layers]}
    return {"layers": layers, "table": table, "out_norm": out_norm, "lm": lm}, om


# ---------------------------------------------------------------- float64 forward
def rms64(v, w, eps):
    return v * w / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + eps)


def rope64(x, pos, hd, theta):
    out = x.copy()
    half = hd // 2
    for h in range(x.size // hd):
        for i in range(half):
            ang = pos / theta ** (2.0 * i / hd)
            a, b = x[h * hd + 2 * i], x[h * hd + 2 * i + 1]
            out[h * hd + 2 * i] = a * np.cos(ang) - b * np.sin(ang)
            out[h * hd + 2 * i + 1] = a * np.sin(ang) + b * np.cos(ang)
    return out


def forward64(m, ids, pos, kc, vc):
    c = CFG
    H, Hkv, hd, eps, theta = c["n_heads"], c["n_kv_heads"], c["head_dim"], c["eps"], c["theta"]
    G = H // Hkv
    f = np.float64
    hidden = m["table"][list(ids)].astype(f)
    layers = m["layers"]
    normed = rms64(hidden, layers[0]["attn_norm"].astype(f), eps)  # ref:src/model.cu:882-885
    kc = [k.astype(f) for k in kc]
    vc = [v.astype(f) for v in vc]
    for i, L in enumerate(layers):
        W = {k: L[k].astype(f) for k in ("q", "k", "v", "o", "gate", "up", "down")}
        q, k, v = normed @ W["q"].T, normed @ W["k"].T, normed @ W["v"].T
        ctx = np.zeros_like(q)
        for t in range(len(ids)):
            qt, kt = rope64(q[t], pos + t, hd, theta), rope64(k[t], pos + t, hd, theta)
            kc[i][pos + t] = kt.reshape(Hkv, hd)
            vc[i][pos + t] = v[t].reshape(Hkv, hd)
        for t in range(len(ids)):
            qt = rope64(q[t], pos + t, hd, theta).reshape(H, hd)
            n = pos + t + 1
            for h in range(H):
                s = kc[i][:n, h // G, :] @ qt[h] / np.sqrt(hd)
                p = np.exp(s - s.max())
                ctx[t, h * hd:(h + 1) * hd] = (p / p.sum()) @ vc[i][:n, h // G, :]
        hidden = hidden + ctx @ W["o"].T  # ref:src/model.cu:963-967
        normed = rms64(hidden, L["ffn_norm"].astype(f), eps)
        g, u = normed @ W["gate"].T, normed @ W["up"].T
        hidden = hidden + ((g / (1 + np.exp(-g))) * u) @ W["down"].T  # ref:src/model.cu:986-1018
        nxt = layers[i + 1]["attn_norm"] if i + 1 < len(layers) else m["out_norm"]
        normed = rms64(hidden, nxt.astype(f), eps)
    lm = m["table"] if m["lm"] is None else m["lm"]  # tied: the FP32 table (ref:src/model.cu:1027-1029)
    return normed @ lm.astype(f).T


def cache(seed, T=32):
    rng = np.random.default_rng(seed)
    shape = (T, CFG["n_kv_heads"], CFG["head_dim"])
    return ([rng.standard_normal(shape).astype(np.float32) for _ in range(CFG["n_layers"])],
            [rng.standard_normal(shape).astype(np.float32) for _ in range(CFG["n_layers"])])


def copies(kc, vc):
    return [k.copy() for k in kc], [v.copy() for v in vc]


@pytest.mark.parametrize("M,pos,tied", [(1, 0, False), (1, 20, False), (3, 7, False), (4, 28, True)])
def test_oracle_step_matches_float64_forward(orc, M, pos, tied):
    m, om = make_model(11 + M + pos, tied)
    kc, vc = cache(5 + pos)
    ids = list(np.random.default_rng(M * 3 + pos).integers(0, CFG["vocab"], M))
    ref = forward64(m, ids, pos, kc, vc)
    got, _ = orc.decode_step(om, ids, pos, *copies(kc, vc))
    err = normwise_rel_err(got, ref)
    print("oracle step M=%d pos=%d tied=%s: %.2e of the float64 forward" % (M, pos, tied, err))
    assert err <= BAR


def _mutated_step(orc, om, ids, pos, kc, vc, mutation):
    """The oracle's composition with one planted mistake, from its own building blocks."""
    eps = om["eps"]
    layers = om["layers"]
    hidden = orc.embed(om, ids)
    if mutation == "no_first_norm":
        normed = hidden.copy()
    else:
        hidden, normed = orc.rmsnorm_residual(hidden, None, layers[0]["attn_norm"], eps)
    for i in range(len(layers)):
        h_in = hidden
        hidden, ffn_out = orc.decode_layer(om, i, hidden, normed, pos, kc[i], vc[i])
        if mutation == "residual_skips_attention":  # the FFN output added to the stream before attention
            hidden = h_in
        if mutation == "same_layer_norm":
            nxt = layers[i]["attn_norm"] if i + 1 < len(layers) else om["out_norm"]
        else:
            nxt = layers[i + 1]["attn_norm"] if i + 1 < len(layers) else om["out_norm"]
        hidden, normed = orc.rmsnorm_residual(hidden, ffn_out, nxt, eps)
    return orc.lm_head(om, normed)[0]


@pytest.mark.parametrize("mutation", ["same_layer_norm", "no_first_norm", "residual_skips_attention"])
def test_planted_composition_mistakes_fail_the_bar(orc, mutation):
    m, om = make_model(77)
    kc, vc = cache(78)
    ids, pos = [3, 9, 41], 10
    ref = forward64(m, ids, pos, kc, vc)
    good = _mutated_step(orc, om, ids, pos, *copies(kc, vc), mutation=None)
    assert normwise_rel_err(good, ref) <= BAR  # the unmutated rebuild passes
    bad = _mutated_step(orc, om, ids, pos, *copies(kc, vc), mutation=mutation)
    err = normwise_rel_err(bad, ref)
    print("planted %s: %.2e of the float64 forward (bar %.0e)" % (mutation, err, BAR))
    assert err > 100 * BAR
