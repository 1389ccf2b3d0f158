"""ctypes binding of the CPU oracle (liboracle.so) plus numpy cross-checks.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.

The C oracle (oracle.c) restates the reference's CPU path; the numpy functions
below restate the *loop-form* CPU references of ref:tests/test_dequantize.cu
independently, so that agreement between the two pins both against the two
formulations the reference itself carries.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

FORMATS = {"q8_0": 0, "q4_0": 1, "q5_0": 2, "q4_k": 3, "q6_k": 4, "fp16": 5}
BLOCK_ELEMS = {"q8_0": 32, "q4_0": 32, "q5_0": 32, "q4_k": 256, "q6_k": 256, "fp16": 1}
BLOCK_BYTES = {"q8_0": 34, "q4_0": 18, "q5_0": 22, "q4_k": 144, "q6_k": 210, "fp16": 2}

_lib = None


def build():
    """Compile liboracle.so with the committed Makefile flags."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        vp, fp, i64, i32 = ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.orc_half_to_float.restype = ctypes.c_float
        L.orc_half_to_float.argtypes = [ctypes.c_uint16]
        L.orc_float_to_half.restype = ctypes.c_uint16
        L.orc_float_to_half.argtypes = [ctypes.c_float]
        for name in ("orc_half_to_float_array", "orc_float_to_half_array"):
            getattr(L, name).argtypes = [vp, vp, i64]
        for f in ("q8_0", "q4_0", "q5_0", "q6_k", "q4_k", "fp16"):
            getattr(L, "orc_dequantize_" + f).argtypes = [vp, fp, i64]
        L.orc_dequantize.argtypes = [i32, vp, fp, i64]
        L.orc_matmul_bt.argtypes = [fp, fp, fp, i32, i32, i32]
        L.orc_matmul_quant_rows.argtypes = [i32, fp, vp, fp, i32, i32, i32, i32, i32]
        L.orc_matmul_quant.argtypes = [i32, fp, vp, fp, i32, i32, i32]
        L.orc_matmul_transposed_b.argtypes = [fp, fp, fp, i32, i32, i32]
        L.orc_batched_matmul_gqa.argtypes = [fp, fp, fp, i32, i32, i32, i32, i32]
        L.orc_rmsnorm_residual.argtypes = [fp, fp, fp, fp, fp, i32, i32, ctypes.c_float]
        L.orc_silu_mul.argtypes = [fp, fp, fp, i64]
        for name in ("orc_decode_attention", "orc_decode_attention_online"):
            getattr(L, name).argtypes = [fp, fp, fp, fp, i32, i32, i32, i32, ctypes.c_float]
        for f in ("q8_0", "q4_0", "q5_0", "q6_k", "q4_k_simple", "q4_k_asym"):
            getattr(L, "orc_quantize_" + f).argtypes = [fp, vp, i64]
        for f in ("q8_0", "q4_0", "q6_k", "q4_k"):
            getattr(L, "orc_make_%s_blocks" % f).argtypes = [vp, i32]
        L.orc_rope.argtypes = [fp, i32, i32, i32, ctypes.c_float]
        L.orc_argmax.argtypes = [fp, i32]
        L.orc_argmax.restype = ctypes.c_int32
        L.orc_random_matrix_lcg.argtypes = [fp, i64, ctypes.c_uint32]
        L.orc_randn.argtypes = [fp, i64, ctypes.c_uint64, ctypes.c_float]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


# ---------------------------------------------------------------- fp16 codec
def half_to_float(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_half_to_float_array(_p(h), _p(out), h.size)
    return out


def float_to_half(f: np.ndarray) -> np.ndarray:
    f = _f32(f)
    out = np.empty(f.shape, np.uint16)
    lib().orc_float_to_half_array(_p(f), _p(out), f.size)
    return out


# ---------------------------------------------------------------- dequant
def dequantize(fmt: str, data: np.ndarray, n_elems: int) -> np.ndarray:
    data = _u8(data)
    assert data.size * BLOCK_ELEMS[fmt] >= n_elems * BLOCK_BYTES[fmt]
    out = np.empty(n_elems, np.float32)
    lib().orc_dequantize(FORMATS[fmt], _p(data), _p(out), n_elems)
    return out


# ---------------------------------------------------------------- matmuls
def matmul_bt(A, B):
    A, B = _f32(A), _f32(B)
    M, K = A.shape
    N = B.shape[0]
    C = np.empty((M, N), np.float32)
    lib().orc_matmul_bt(_p(A), _p(B), _p(C), M, N, K)
    return C


def matmul_quant(fmt: str, A, Bq, N: int, K: int, rows=None):
    """C = A * dequant(Bq)^T; if rows=(n0, n1) only those output columns are filled."""
    A, Bq = _f32(A), _u8(Bq)
    M = A.shape[0]
    C = np.zeros((M, N), np.float32)
    n0, n1 = (0, N) if rows is None else rows
    lib().orc_matmul_quant_rows(FORMATS[fmt], _p(A), _p(Bq), _p(C), M, N, K, n0, n1)
    return C


def matmul_quant_mt(fmt: str, A, Bq, N: int, K: int, threads=None):
    """matmul_quant with the output columns split over threads (each thread runs the same
    sequential per-element arithmetic on its own columns, so the result is bit-identical)."""
    import concurrent.futures as cf

    A, Bq = _f32(A), _u8(Bq)
    M = A.shape[0]
    C = np.zeros((M, N), np.float32)
    threads = threads or min(16, os.cpu_count() or 4)
    step = max(1, -(-N // threads))
    L = lib()

    def run(n0):
        L.orc_matmul_quant_rows(FORMATS[fmt], _p(A), _p(Bq), _p(C), M, N, K, n0, min(N, n0 + step))

    with cf.ThreadPoolExecutor(threads) as ex:
        list(ex.map(run, range(0, N, step)))
    return C


def matmul_transposed_b(A, B):
    A, B = _f32(A), _f32(B)
    M, K = A.shape
    N = B.shape[0]
    C = np.empty((M, N), np.float32)
    lib().orc_matmul_transposed_b(_p(A), _p(B), _p(C), M, N, K)
    return C


def batched_matmul_gqa(A, B, n_heads, n_kv_heads, M, N, K):
    A, B = _f32(A), _f32(B)
    C = np.empty((n_heads, M, N), np.float32)
    lib().orc_batched_matmul_gqa(_p(A), _p(B), _p(C), n_heads, n_kv_heads, M, N, K)
    return C


def decode_attention(Q, K, V, n_heads, n_kv_heads, head_dim, kv_len, scale, online=False):
    """One-token attention over the [kv_len, n_kv_heads, head_dim] cache: the
    reference CPU test's two-pass softmax, or (online=True) the reference kernel's
    single-pass recurrence.  K and V may hold more positions than kv_len."""
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    assert Q.size >= n_heads * head_dim and K.size >= kv_len * n_kv_heads * head_dim
    assert V.size >= kv_len * n_kv_heads * head_dim
    out = np.empty(n_heads * head_dim, np.float32)
    fn = lib().orc_decode_attention_online if online else lib().orc_decode_attention
    fn(_p(Q), _p(K), _p(V), _p(out), n_heads, n_kv_heads, head_dim, kv_len, float(scale))
    return out


def np_decode_attention_f64(Q, K, V, n_heads, n_kv_heads, head_dim, kv_len, scale):
    """fp64 brute force of the same attention (numpy, independent of the C code)."""
    G = n_heads // n_kv_heads
    q = np.asarray(Q, np.float64).reshape(n_heads, head_dim)
    k = np.asarray(K, np.float64).reshape(-1, n_kv_heads, head_dim)[:kv_len]
    v = np.asarray(V, np.float64).reshape(-1, n_kv_heads, head_dim)[:kv_len]
    out = np.empty((n_heads, head_dim))
    for h in range(n_heads):
        s = k[:, h // G, :] @ q[h] * float(np.float32(scale))
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ v[:, h // G, :]
    return out.ravel()


def rmsnorm_residual(x, residual, weight, eps=1e-5):
    """(output, normed) of the reference's rmsnorm_residual over rows of x [rows, n]."""
    x = _f32(x)
    rows, n = x.shape
    res = None if residual is None else _f32(residual).reshape(rows, n)
    w = _f32(weight)
    out = np.empty_like(x)
    normed = np.empty_like(x)
    lib().orc_rmsnorm_residual(_p(x), None if res is None else _p(res), _p(w), _p(out), _p(normed), rows, n,
                               float(eps))
    return out, normed


def silu_mul(gate, up):
    g, u = _f32(gate), _f32(up)
    out = np.empty_like(g)
    lib().orc_silu_mul(_p(g), _p(u), _p(out), g.size)
    return out


def rope(x, pos, head_dim, n_heads, theta):
    """RoPE of one token's heads (ref:src/kernels/elementwise.cu:232-257); returns a copy."""
    out = _f32(x).copy()
    lib().orc_rope(_p(out), int(pos), head_dim, n_heads, float(theta))
    return out


def argmax(x):
    """The reference kernel's argmax (ref:src/embedding.cu:155-200)."""
    x = _f32(x)
    return int(lib().orc_argmax(_p(x), x.size))


def _mm(w, x, N, K):
    fmt, data = w
    return matmul_quant_mt(fmt, x, data, N, K)


def embed(model, ids):
    """The token rows of the step's input (ref:src/embedding.cu:237-263 reads an FP32 table; a
    quantized table's row is its blocks dequantized: dequantize + gather)."""
    V, dim = model["vocab"], model["dim"]
    tfmt, table = model["tok"]
    if tfmt == "fp32":
        return _f32(np.asarray(table, np.float32).reshape(V, dim)[list(ids)])
    rb = dim // BLOCK_ELEMS[tfmt] * BLOCK_BYTES[tfmt]
    t = _u8(table)
    return np.stack([dequantize(tfmt, t[i * rb:(i + 1) * rb], dim) for i in ids])


def decode_layer(model, i, hidden, normed, pos, k_cache, v_cache):
    """Layer i of the reference's quantized forward pass (ref:src/model.cu:887-1019) on the
    residual stream `hidden` [M, dim] and its RMSNorm `normed` (with layer i's attn_norm), at
    positions pos .. pos + M - 1.  k_cache / v_cache: this layer's [max_seq, n_kv_heads,
    head_dim] arrays, appended to in place.  Returns (hidden + attention + FFN output: the
    stream entering layer i + 1, before its norm; the FFN output)."""
    H, Hkv, D = model["n_heads"], model["n_kv_heads"], model["head_dim"]
    dim, F = model["dim"], model["ffn"]
    eps, theta = model["eps"], model["theta"]
    M = hidden.shape[0]
    qd, kvd = H * D, Hkv * D
    L = model["layers"][i]
    scale = np.float32(1.0) / np.float32(np.sqrt(np.float32(D)))
    q = _mm(L["q"], normed, qd, dim)  # ref:src/model.cu:910-918
    k = _mm(L["k"], normed, kvd, dim)
    v = _mm(L["v"], normed, kvd, dim)
    for t in range(M):  # ref:src/model.cu:921-926
        q[t] = rope(q[t], pos + t, D, H, theta)
        k[t] = rope(k[t], pos + t, D, Hkv, theta)
    k_cache[pos:pos + M] = k.reshape(M, Hkv, D)  # KVCache::append, ref:src/kv_cache.cu:157-211
    v_cache[pos:pos + M] = v.reshape(M, Hkv, D)
    ctx = np.stack([decode_attention(q[t], k_cache, v_cache, H, Hkv, D, pos + t + 1, scale)
                    for t in range(M)])  # row t sees positions <= pos + t (ref:src/attention.cu:60-75)
    attn_out = _mm(L["o"], ctx, dim, qd)
    hidden, normed = rmsnorm_residual(hidden, attn_out, L["ffn_norm"], eps)  # ref:src/model.cu:963-967
    gate = _mm(L["gate"], normed, F, dim)  # ref:src/model.cu:986-994
    up = _mm(L["up"], normed, F, dim)
    act = silu_mul(gate, up)  # ref:src/model.cu:996-997
    ffn_out = _mm(L["down"], act, dim, F)
    return hidden, ffn_out


def lm_head(model, normed):
    """Logits of the final-normed rows (ref:src/model.cu:1023-1037; a tied FP32 table through
    matmul_transposed_b, ref:src/model.cu:1027-1029) and their argmax ids."""
    V, dim = model["vocab"], model["dim"]
    lm = model["lm"] if model["lm"] is not None else model["tok"]
    if lm[0] == "fp32":
        logits = matmul_transposed_b(normed, np.asarray(lm[1], np.float32).reshape(V, dim))
    else:
        logits = _mm(lm, normed, V, dim)
    return logits, np.array([argmax(r) for r in logits], np.int32)


def decode_step(model, ids, pos, k_cache, v_cache):
    """One forward of the tokens `ids` at positions pos .. pos + M - 1, composed from
    the oracle's functions in the order of the reference's quantized forward pass
    (ref:src/model.cu:876-1039).  `model`: dict with n_heads, n_kv_heads, head_dim,
    dim, ffn, vocab, eps, theta, 'tok' (fmt, table bytes or fp32 [vocab, dim]),
    'layers' (list of dicts: attn_norm, ffn_norm and (fmt, bytes) for q, k, v, o,
    gate, up, down), 'out_norm' and 'lm' ((fmt, bytes), or None for a head tied to
    the token table).  k_cache / v_cache: one [max_seq, n_kv_heads, head_dim] fp32
    array per layer, appended to in place.  Returns (logits [M, vocab], argmax ids)."""
    eps = model["eps"]
    layers = model["layers"]
    hidden = embed(model, ids)
    # first layer's standalone RMSNorm (ref:src/model.cu:882-885)
    hidden, normed = rmsnorm_residual(hidden, None, layers[0]["attn_norm"], eps)
    for i in range(len(layers)):
        hidden, ffn_out = decode_layer(model, i, hidden, normed, pos, k_cache[i], v_cache[i])
        nxt = layers[i + 1]["attn_norm"] if i + 1 < len(layers) else model["out_norm"]
        hidden, normed = rmsnorm_residual(hidden, ffn_out, nxt, eps)  # ref:src/model.cu:1008-1018
    return lm_head(model, normed)


# ---------------------------------------------------------------- quantizers
def quantize(fmt: str, x) -> np.ndarray:
    """Host quantizers restated from ref:tests/test_matmul_quant.cu.
    fmt 'q4_k' is the reference's simplified quantizer; 'q4_k_asym' is own."""
    x = _f32(x).ravel()
    name = {"q4_k": "q4_k_simple"}.get(fmt, fmt)
    base = "q4_k" if fmt.startswith("q4_k") else fmt
    nb = x.size // BLOCK_ELEMS[base]
    out = np.zeros(nb * BLOCK_BYTES[base], np.uint8)
    getattr(lib(), "orc_quantize_" + name)(_p(x), _p(out), x.size)
    return out


def make_blocks(fmt: str, n_blocks: int) -> np.ndarray:
    out = np.zeros(n_blocks * BLOCK_BYTES[fmt], np.uint8)
    getattr(lib(), "orc_make_%s_blocks" % fmt)(_p(out), n_blocks)
    return out


def random_matrix_lcg(rows, cols, seed=42):
    out = np.empty(rows * cols, np.float32)
    lib().orc_random_matrix_lcg(_p(out), out.size, seed)
    return out.reshape(rows, cols)


def randn(n, seed, sigma=1.0):
    out = np.empty(n, np.float32)
    lib().orc_randn(_p(out), n, seed, sigma)
    return out


# ------------------------------------------------- numpy loop-form references
def np_dequant_q6_k_loopform(data: np.ndarray) -> np.ndarray:
    """ref:tests/test_dequantize.cu:54-80, vectorised over blocks (own numpy)."""
    blk = _u8(data).reshape(-1, 210)
    d = blk[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    sc = blk[:, 192:208].view(np.int8).astype(np.float32)
    out = np.empty((blk.shape[0], 256), np.float32)
    for n in (0, 128):
        ql = blk[:, (n // 128) * 64:(n // 128) * 64 + 64].astype(np.int32)
        qh = blk[:, 128 + (n // 128) * 32:128 + (n // 128) * 32 + 32].astype(np.int32)
        l = np.arange(32)
        is_ = n // 16 + l // 16
        q1 = ((ql[:, l] & 0xF) | (((qh[:, l] >> 0) & 3) << 4)) - 32
        q2 = ((ql[:, l + 32] & 0xF) | (((qh[:, l] >> 2) & 3) << 4)) - 32
        q3 = ((ql[:, l] >> 4) | (((qh[:, l] >> 4) & 3) << 4)) - 32
        q4 = ((ql[:, l + 32] >> 4) | (((qh[:, l] >> 6) & 3) << 4)) - 32
        for off, q, s in ((0, q1, 0), (32, q2, 2), (64, q3, 4), (96, q4, 6)):
            out[:, n + off + l] = (d[:, None] * sc[:, is_ + s]) * q.astype(np.float32)
    return out.ravel()


def np_dequant_q4_k_loopform(data: np.ndarray) -> np.ndarray:
    """ref:tests/test_dequantize.cu:85-131, vectorised over blocks (own numpy)."""
    blk = _u8(data).reshape(-1, 144)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = blk[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    s = blk[:, 4:16].astype(np.int32)
    q = blk[:, 16:144].astype(np.int32)

    def scale_min(j):
        if j < 4:
            return s[:, j] & 63, s[:, j + 4] & 63
        return (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4), (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)

    out = np.empty((blk.shape[0], 256), np.float32)
    for c in range(4):
        sc1, m1 = scale_min(2 * c)
        sc2, m2 = scale_min(2 * c + 1)
        d1 = d * sc1.astype(np.float32)
        mm1 = dmin * m1.astype(np.float32)
        d2 = d * sc2.astype(np.float32)
        mm2 = dmin * m2.astype(np.float32)
        qq = q[:, 32 * c:32 * c + 32]
        out[:, 64 * c:64 * c + 32] = d1[:, None] * (qq & 0xF).astype(np.float32) - mm1[:, None]
        out[:, 64 * c + 32:64 * c + 64] = d2[:, None] * (qq >> 4).astype(np.float32) - mm2[:, None]
    return out.ravel()


def np_dequant_simple(fmt: str, data: np.ndarray) -> np.ndarray:
    """Vectorised numpy restatement of the 32-element formats (own code, from
    ref:tests/test_dequantize.cu:23-49 and ref:tests/test_matmul_quant.cu:464-487)."""
    bb = BLOCK_BYTES[fmt]
    blk = _u8(data).reshape(-1, bb)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0][:, None]
    if fmt == "q8_0":
        q = blk[:, 2:34].view(np.int8).astype(np.float32)
    elif fmt == "q4_0":
        qs = blk[:, 2:18].astype(np.int32)
        q = np.empty((blk.shape[0], 32), np.int32)
        q[:, 0::2] = qs & 0xF
        q[:, 1::2] = qs >> 4
        q = (q - 8).astype(np.float32)
    elif fmt == "q5_0":
        qh = blk[:, 2:6].copy().view("<u4").astype(np.int64)  # [nb, 1]
        qs = blk[:, 6:22].astype(np.int64)
        low = np.concatenate([qs & 0xF, qs >> 4], axis=1)
        hb = (qh >> np.arange(32)[None, :]) & 1
        q = ((low | (hb << 4)) - 16).astype(np.float32)
    else:
        raise ValueError(fmt)
    return (d * q).ravel()


def np_matmul_f64(A, W):
    """fp64 brute force C = A W^T."""
    return np.asarray(A, np.float64) @ np.asarray(W, np.float64).T
