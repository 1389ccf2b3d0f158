"""Vectorised host quantizers for synthetic GGUF weights (numpy).

These produce the packed block bytes the kernels consume; they are data
generators, not part of the timed path.  Q8_0, Q4_0, Q5_0 and Q6_K follow the
reference's host quantizers (ref:tests/test_matmul_quant.cu:46-71, 74-102,
410-460, 611-686) operation for operation in binary32, so their bytes are
identical to a scalar restatement; Q4_K uses an asymmetric quantizer (nonzero
dmin and mins, which the reference's simplified one at :107-184 never sets).

Rounding: std::round is half-away-from-zero; __float2half is
round-to-nearest-even (numpy's float32 -> float16 cast).
"""
from __future__ import annotations

import numpy as np

BLOCK_ELEMS = {"q8_0": 32, "q4_0": 32, "q5_0": 32, "q4_k": 256, "q6_k": 256, "fp16": 1, "fp32": 1}
BLOCK_BYTES = {"q8_0": 34, "q4_0": 18, "q5_0": 22, "q4_k": 144, "q6_k": 210, "fp16": 2, "fp32": 4}
FORMAT_IDS = {"q8_0": 0, "q4_0": 1, "q5_0": 2, "q4_k": 3, "q6_k": 4, "fp16": 5}

F32 = np.float32


def row_bytes(fmt: str, K: int) -> int:
    return (K // BLOCK_ELEMS[fmt]) * BLOCK_BYTES[fmt]


def _roundf(v: np.ndarray) -> np.ndarray:
    """C roundf: nearest, ties away from zero (exact for binary32 inputs)."""
    t = np.trunc(v)
    frac = v - t  # exact
    return t + np.where(np.abs(frac) >= F32(0.5), np.sign(v), F32(0)).astype(v.dtype)


def _to_int(v: np.ndarray) -> np.ndarray:
    return _roundf(v).astype(np.int64)


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return v.astype(np.float16).view(np.uint8).reshape(v.shape[0], 2)


def _f16_round(v: np.ndarray) -> np.ndarray:
    return v.astype(np.float16).astype(F32)


def _amax(xb: np.ndarray) -> np.ndarray:
    return np.max(np.abs(xb), axis=1)


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    xb = np.ascontiguousarray(x, F32).reshape(-1, 32)
    scale = _amax(xb) / F32(127.0)
    scale[scale == 0] = F32(1.0)
    inv = F32(1.0) / scale
    q = np.clip(_to_int(xb * inv[:, None]), -128, 127).astype(np.int8)
    out = np.empty((xb.shape[0], 34), np.uint8)
    out[:, 0:2] = _f16_bytes(scale)
    out[:, 2:] = q.view(np.uint8)
    return out.ravel()


def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    xb = np.ascontiguousarray(x, F32).reshape(-1, 32)
    scale = _amax(xb) / F32(8.0)
    scale[scale == 0] = F32(1.0)
    inv = F32(1.0) / scale
    q = np.clip(_to_int(xb * inv[:, None]) + 8, 0, 15).astype(np.uint8)
    out = np.empty((xb.shape[0], 18), np.uint8)
    out[:, 0:2] = _f16_bytes(scale)
    out[:, 2:] = q[:, 0::2] | (q[:, 1::2] << 4)  # element i -> qs[i/2], low nibble for even i
    return out.ravel()


def quantize_q5_0(x: np.ndarray) -> np.ndarray:
    xb = np.ascontiguousarray(x, F32).reshape(-1, 32)
    scale = _amax(xb) / F32(16.0)
    scale[scale == 0] = F32(1.0)
    inv = F32(1.0) / scale
    q = np.clip(_to_int(xb * inv[:, None]) + 16, 0, 31).astype(np.uint32)
    low = (q & 0xF).astype(np.uint8)
    hb = (q >> 4) & 1
    qh = np.sum(hb << np.arange(32, dtype=np.uint32)[None, :], axis=1, dtype=np.uint64).astype("<u4")
    out = np.empty((xb.shape[0], 22), np.uint8)
    out[:, 0:2] = _f16_bytes(scale)
    out[:, 2:6] = qh.view(np.uint8).reshape(-1, 4)
    out[:, 6:] = low[:, :16] | (low[:, 16:] << 4)
    return out.ravel()


def quantize_q6_k(x: np.ndarray) -> np.ndarray:
    xb = np.ascontiguousarray(x, F32).reshape(-1, 256)
    nb = xb.shape[0]
    amax = _amax(xb)
    sub_amax = np.max(np.abs(xb.reshape(nb, 16, 16)), axis=2)
    d = np.where(amax > 0, amax / F32(32.0 * 31.0), F32(1.0)).astype(F32)
    inv_d = F32(1.0) / d
    sub_scale = np.where(sub_amax > 0, sub_amax / F32(31.0), F32(0.0)).astype(F32)
    sc = np.clip(_to_int(sub_scale * inv_d[:, None]).astype(np.int8).astype(np.int64), -127, 127)
    eff = (d[:, None] * sc.astype(F32)).astype(F32)  # [nb, 16]
    with np.errstate(divide="ignore"):
        inv_eff = np.where(eff != 0, F32(1.0) / np.where(eff != 0, eff, F32(1.0)), F32(0.0)).astype(F32)
    inv_e = np.repeat(inv_eff, 16, axis=1)  # per element
    q6 = np.clip(_to_int(xb * inv_e) + 32, 0, 63).astype(np.uint8)  # [nb, 256]
    out = np.zeros((nb, 210), np.uint8)
    for c in range(2):
        base = q6[:, 128 * c:128 * c + 128]
        quarters = [base[:, 32 * qq:32 * qq + 32] for qq in range(4)]
        low = [qq & 0xF for qq in quarters]
        high = [(qq >> 4) & 3 for qq in quarters]
        out[:, 64 * c:64 * c + 32] = low[0] | (low[2] << 4)
        out[:, 64 * c + 32:64 * c + 64] = low[1] | (low[3] << 4)
        out[:, 128 + 32 * c:128 + 32 * c + 32] = high[0] | (high[1] << 2) | (high[2] << 4) | (high[3] << 6)
    out[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    out[:, 208:210] = _f16_bytes(d)
    return out.ravel()


def quantize_q4_k(x: np.ndarray) -> np.ndarray:
    """Asymmetric Q4_K: x ~= d*sc*q - dmin*mn per 32-element sub-block (own scheme)."""
    xb = np.ascontiguousarray(x, F32).reshape(-1, 256)
    nb = xb.shape[0]
    sub = xb.reshape(nb, 8, 32)
    lo = np.minimum(np.min(sub, axis=2), F32(0.0))
    hi = np.max(sub, axis=2)
    sub_scale = ((hi - lo) / F32(15.0)).astype(F32)
    sub_min = (-lo).astype(F32)
    # running maxima start from +0 (so an all -0 set of offsets gives +0, not -0)
    d = (np.max(np.where(sub_scale > 0, sub_scale, F32(0.0)), axis=1) / F32(63.0)).astype(F32)
    dmin = (np.max(np.where(sub_min > 0, sub_min, F32(0.0)), axis=1) / F32(63.0)).astype(F32)
    with np.errstate(divide="ignore"):
        inv_d = np.where(d > 0, F32(1.0) / np.where(d > 0, d, F32(1.0)), F32(0.0)).astype(F32)
        inv_m = np.where(dmin > 0, F32(1.0) / np.where(dmin > 0, dmin, F32(1.0)), F32(0.0)).astype(F32)
    sc = np.clip(_to_int(sub_scale * inv_d[:, None]), 0, 63)
    mn = np.clip(_to_int(sub_min * inv_m[:, None]), 0, 63)
    dq, dmq = _f16_round(d), _f16_round(dmin)
    eff = (dq[:, None] * sc.astype(F32)).astype(F32)
    off = (dmq[:, None] * mn.astype(F32)).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        qv = (sub + off[:, :, None]) / np.where(eff > 0, eff, F32(1.0))[:, :, None]
    q = np.where(eff[:, :, None] > 0, np.clip(_to_int(qv.astype(F32)), 0, 15), 0).astype(np.uint8)
    q = q.reshape(nb, 256)
    out = np.zeros((nb, 144), np.uint8)
    out[:, 0:2] = _f16_bytes(d)
    out[:, 2:4] = _f16_bytes(dmin)
    s = np.zeros((nb, 12), np.int64)
    for j in range(4):
        s[:, j] = (sc[:, j] & 0x3F) | ((sc[:, j + 4] >> 4) << 6)
        s[:, j + 4] = (mn[:, j] & 0x3F) | ((mn[:, j + 4] >> 4) << 6)
        s[:, j + 8] = (sc[:, j + 4] & 0x0F) | ((mn[:, j + 4] & 0x0F) << 4)
    out[:, 4:16] = s.astype(np.uint8)
    for c in range(4):
        out[:, 16 + 32 * c:16 + 32 * c + 32] = q[:, 64 * c:64 * c + 32] | (q[:, 64 * c + 32:64 * c + 64] << 4)
    return out.ravel()


def quantize_fp16(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, F32).astype(np.float16).view(np.uint8).ravel()


QUANTIZERS = {
    "q8_0": quantize_q8_0,
    "q4_0": quantize_q4_0,
    "q5_0": quantize_q5_0,
    "q4_k": quantize_q4_k,
    "q6_k": quantize_q6_k,
    "fp16": quantize_fp16,
}


def quantize(fmt: str, x: np.ndarray) -> np.ndarray:
    return QUANTIZERS[fmt](x)


def randn(n: int, seed: int, sigma: float = 1.0) -> np.ndarray:
    """N(0, sigma^2) float32 synthetic data (numpy PCG64)."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(n, dtype=np.float32) * F32(sigma)).astype(F32)


def synthetic_weights(fmt: str, N: int, K: int, seed: int, sigma: float = 0.02, chunk_rows: int = 4096) -> np.ndarray:
    """w ~ N(0, sigma^2) of shape [N, K], quantised row-chunk by row-chunk."""
    rb = row_bytes(fmt, K)
    out = np.empty(N * rb, np.uint8)
    rng = np.random.default_rng(seed)
    for r0 in range(0, N, chunk_rows):
        r1 = min(N, r0 + chunk_rows)
        w = (rng.standard_normal((r1 - r0) * K, dtype=np.float32) * F32(sigma)).astype(F32)
        out[r0 * rb:r1 * rb] = quantize(fmt, w)
    return out


# fp16 scale fields of random_blocks: weights of standard deviation ~0.02, as N(0, 0.02) weights
RANDOM_BLOCK_SCALE = {"q8_0": 2.6e-4, "q4_0": 4.3e-3, "q5_0": 2.2e-3, "q4_k": 1e-4, "q6_k": 1.5e-5, "fp16": 3.5e-4}


def random_blocks(fmt: str, N: int, K: int, seed: int, scale: float | None = None) -> np.ndarray:
    """[N, K] weights as uniformly random block bytes with every fp16 scale field set to
    `scale` times a factor in [0.5, 1.5): valid blocks of every code, ~100x faster to make
    than quantized Gaussians.  For parity tests at full model size (both sides read the
    same bytes), not for measurements."""
    scale = RANDOM_BLOCK_SCALE[fmt] if scale is None else scale
    rb = row_bytes(fmt, K)
    rng = np.random.default_rng(seed)
    out = rng.integers(0, 256, size=N * rb, dtype=np.uint8)
    if fmt == "fp16":
        v = (rng.random(N * K, dtype=np.float32) - F32(0.5)) * F32(200.0 * scale)
        return v.astype(np.float16).view(np.uint8)
    blk = out.reshape(-1, BLOCK_BYTES[fmt])

    def f16(n):
        return (F32(scale) * (F32(0.5) + rng.random(n, dtype=np.float32))).astype(np.float16).view(np.uint8).reshape(
            n, 2)

    nb = blk.shape[0]
    if fmt in ("q8_0", "q4_0", "q5_0"):
        blk[:, 0:2] = f16(nb)
    elif fmt == "q4_k":  # d, dmin
        blk[:, 0:2] = f16(nb)
        blk[:, 2:4] = f16(nb)
    elif fmt == "q6_k":  # d is the last field
        blk[:, 208:210] = f16(nb)
    else:
        raise ValueError(fmt)
    return out
