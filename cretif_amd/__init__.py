"""cretif_amd -- MI355X (gfx950) fused dequant+matmul over GGUF block layouts.

Python mirror of the reference's operator interface for this path.  Every
function takes the reference's arguments in the reference's order
(ref:include/cuinfer/kernels/matmul_quant.h:37-105,
ref:include/cuinfer/quantization.h:145-174, ref:include/cuinfer/embedding.h:136,
ref:include/cuinfer/attention.h:79-82) and calls the C ABI of libcretif.so
(include/cri.h) directly.  Buffers are device tensors (torch, on the GPU) or
raw device addresses (int); nothing is copied or allocated here.  Failures
raise CretifError, as the reference's C++ entry points throw
std::runtime_error.

There is no CPU fallback: if libcretif.so is missing or no GPU is present,
the call raises.
"""
from __future__ import annotations

import ctypes
import os

__all__ = [
    "CretifError",
    "lib",
    "library_path",
    "matmul",
    "matmul_q8_0",
    "matmul_q4_0",
    "matmul_q5_0",
    "matmul_q4_k",
    "matmul_q6_k",
    "matmul_fp16",
    "dequantize",
    "dequantize_q8_0",
    "dequantize_q4_0",
    "dequantize_q5_0",
    "dequantize_q6_k",
    "dequantize_q4_k",
    "matmul_transposed_b",
    "batched_matmul_gqa",
    "fused_decode_attention",
    "fused_decode_attention_ws",
    "decode_attention_workspace_size",
    "matmul_rmsnorm",
    "matmul_swiglu",
    "rmsnorm_residual",
    "silu_mul",
    "FORMAT_IDS",
    "ABI_SYMBOLS",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
library_path = os.path.join(_HERE, "libcretif.so")

FORMAT_IDS = {"q8_0": 0, "q4_0": 1, "q5_0": 2, "q4_k": 3, "q6_k": 4, "fp16": 5}
STATUS_NAMES = {
    0: "CRI_OK",
    -1: "CRI_ERR_INVALID_ARGUMENT",
    -2: "CRI_ERR_SHAPE",
    -3: "CRI_ERR_ALIGNMENT",
    -4: "CRI_ERR_LAUNCH",
    -5: "CRI_ERR_UNSUPPORTED",
}

_MATMUL = ["cri_matmul_" + f for f in ("q8_0", "q4_0", "q5_0", "q4_k", "q6_k", "fp16")]
_DEQUANT = ["cri_dequantize_" + f for f in ("q8_0", "q4_0", "q5_0", "q6_k", "q4_k")]
ABI_SYMBOLS = (
    _MATMUL
    + ["cri_matmul"]
    + _DEQUANT
    + [
        "cri_matmul_transposed_b",
        "cri_batched_matmul_gqa",
        "cri_fused_decode_attention",
        "cri_fused_decode_attention_ws",
        "cri_fused_decode_attention_workspace_size",
        "cri_matmul_rmsnorm",
        "cri_matmul_swiglu",
        "cri_rmsnorm_residual",
        "cri_silu_mul",
        "cri_last_error_string",
        "cri_block_bytes",
        "cri_block_elems",
        "cri_version",
    ]
)


class CretifError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__("%s (%d): %s" % (STATUS_NAMES.get(status, "?"), status, message))
        self.status = status


_lib = None


def lib():
    """Load libcretif.so (after torch, so both share torch's HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(library_path):
        raise RuntimeError("libcretif.so is not built; run `python -m cretif_amd.build` (or __graft_entry__.build())")
    try:
        import torch  # noqa: F401  -- load torch's libamdhip64 first so there is one HIP runtime
    except ImportError:
        pass
    L = ctypes.CDLL(library_path)
    vp, i32 = ctypes.c_void_p, ctypes.c_int
    for name in _MATMUL:
        f = getattr(L, name)
        f.argtypes = [vp, vp, vp, i32, i32, i32, vp]
        f.restype = i32
    L.cri_matmul.argtypes = [i32, vp, vp, vp, i32, i32, i32, vp]
    L.cri_matmul.restype = i32
    for name in _DEQUANT:
        f = getattr(L, name)
        f.argtypes = [vp, vp, i32, vp]
        f.restype = i32
    L.cri_matmul_transposed_b.argtypes = [vp, vp, vp, i32, i32, i32, vp]
    L.cri_matmul_transposed_b.restype = i32
    L.cri_batched_matmul_gqa.argtypes = [vp, vp, vp, i32, i32, i32, i32, i32, vp]
    L.cri_batched_matmul_gqa.restype = i32
    L.cri_fused_decode_attention.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, ctypes.c_float, vp]
    L.cri_fused_decode_attention.restype = i32
    L.cri_fused_decode_attention_ws.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, ctypes.c_float, vp,
                                                 ctypes.c_longlong, vp]
    L.cri_fused_decode_attention_ws.restype = i32
    L.cri_fused_decode_attention_workspace_size.argtypes = [i32, i32, i32, i32]
    L.cri_fused_decode_attention_workspace_size.restype = ctypes.c_longlong
    L.cri_matmul_rmsnorm.argtypes = [i32, vp, vp, vp, vp, vp, vp, i32, i32, i32, ctypes.c_float, vp]
    L.cri_matmul_rmsnorm.restype = i32
    L.cri_matmul_swiglu.argtypes = [i32, vp, vp, i32, vp, vp, i32, i32, i32, vp]
    L.cri_matmul_swiglu.restype = i32
    L.cri_rmsnorm_residual.argtypes = [vp, vp, vp, vp, vp, i32, i32, ctypes.c_float, vp]
    L.cri_rmsnorm_residual.restype = i32
    L.cri_silu_mul.argtypes = [vp, vp, vp, ctypes.c_longlong, vp]
    L.cri_silu_mul.restype = i32
    L.cri_last_error_string.argtypes = []
    L.cri_last_error_string.restype = ctypes.c_char_p
    L.cri_block_bytes.argtypes = [i32]
    L.cri_block_bytes.restype = i32
    L.cri_block_elems.argtypes = [i32]
    L.cri_block_elems.restype = i32
    L.cri_version.restype = i32
    _lib = L
    return L


def _ptr(t):
    """Device address of a torch tensor (must live on the GPU) or a raw int."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    dev = getattr(t, "device", None)
    if dev is None:
        raise TypeError("expected a device tensor or an int address, got %r" % type(t))
    if dev.type != "cuda":
        raise ValueError("buffer is on %s; the HIP kernels need device (cuda) tensors" % dev)
    if not t.is_contiguous():
        raise ValueError("buffer must be contiguous")
    return t.data_ptr()


def _stream(stream):
    if stream is None:
        import torch

        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream  # torch.cuda.Stream


def _check(status: int):
    if status != 0:
        msg = lib().cri_last_error_string().decode("utf-8", "replace")
        raise CretifError(status, msg)


def _mm(name):
    def fn(A, B, C, M, N, K, stream=None):
        _check(getattr(lib(), "cri_" + name)(_ptr(A), _ptr(B), _ptr(C), M, N, K, _stream(stream)))

    fn.__name__ = name
    fn.__doc__ = "C[M,N] = A[M,K] * dequant(B[N,K])^T (replaces cuinfer::%s)." % name
    return fn


matmul_q8_0 = _mm("matmul_q8_0")
matmul_q4_0 = _mm("matmul_q4_0")
matmul_q5_0 = _mm("matmul_q5_0")
matmul_q4_k = _mm("matmul_q4_k")
matmul_q6_k = _mm("matmul_q6_k")
matmul_fp16 = _mm("matmul_fp16")


def matmul(fmt, A, B, C, M, N, K, stream=None):
    """Format-switched fused matmul (the switch of matmul_dispatch, ref:src/model.cu:797-825)."""
    fid = FORMAT_IDS[fmt] if isinstance(fmt, str) else int(fmt)
    _check(lib().cri_matmul(fid, _ptr(A), _ptr(B), _ptr(C), M, N, K, _stream(stream)))


def _dq(name):
    def fn(src, dst, n_blocks, stream=None):
        _check(getattr(lib(), "cri_" + name)(_ptr(src), _ptr(dst), n_blocks, _stream(stream)))

    fn.__name__ = name
    fn.__doc__ = "dst[n_blocks * block] = dequant(src) (replaces cuinfer::%s)." % name
    return fn


dequantize_q8_0 = _dq("dequantize_q8_0")
dequantize_q4_0 = _dq("dequantize_q4_0")
dequantize_q5_0 = _dq("dequantize_q5_0")
dequantize_q6_k = _dq("dequantize_q6_k")
dequantize_q4_k = _dq("dequantize_q4_k")


def dequantize(fmt, src, dst, n_blocks, stream=None):
    {
        "q8_0": dequantize_q8_0,
        "q4_0": dequantize_q4_0,
        "q5_0": dequantize_q5_0,
        "q6_k": dequantize_q6_k,
        "q4_k": dequantize_q4_k,
    }[fmt](src, dst, n_blocks, stream)


def matmul_transposed_b(A, B, C, M, N, K, stream=None):
    """C[M,N] = A[M,K] * B[N,K]^T, fp32 (replaces cuinfer::matmul_transposed_b)."""
    _check(lib().cri_matmul_transposed_b(_ptr(A), _ptr(B), _ptr(C), M, N, K, _stream(stream)))


def batched_matmul_gqa(A, B, C, n_heads, n_kv_heads, M, N, K, stream=None):
    """C[h] = A[h] * B[h / (n_heads/n_kv_heads)] (replaces cuinfer::batched_matmul_gqa)."""
    _check(
        lib().cri_batched_matmul_gqa(
            _ptr(A), _ptr(B), _ptr(C), n_heads, n_kv_heads, M, N, K, _stream(stream)
        )
    )


def fused_decode_attention(Q, K_cache, V_cache, output, n_heads, n_kv_heads, head_dim, kv_len, scale, stream=None):
    """output[h] = softmax(scale * Q[h] . K[t, h/G]) V[t, h/G] over t < kv_len, one query token
    (replaces cuinfer::fused_decode_attention, ref:include/cuinfer/attention.h:161-167)."""
    _check(
        lib().cri_fused_decode_attention(
            _ptr(Q),
            _ptr(K_cache),
            _ptr(V_cache),
            _ptr(output),
            n_heads,
            n_kv_heads,
            head_dim,
            kv_len,
            float(scale),
            _stream(stream),
        )
    )


def decode_attention_workspace_size(n_heads, n_kv_heads, head_dim, kv_len):
    """Bytes of device workspace fused_decode_attention_ws uses for this shape."""
    n = lib().cri_fused_decode_attention_workspace_size(n_heads, n_kv_heads, head_dim, kv_len)
    if n < 0:
        _check(int(n))
    return int(n)


def fused_decode_attention_ws(Q, K_cache, V_cache, output, n_heads, n_kv_heads, head_dim, kv_len, scale,
                              workspace, workspace_bytes=None, stream=None):
    """Split form of fused_decode_attention with partial results in a caller
    workspace (a device tensor, or an address plus workspace_bytes).  No
    counterpart in the reference."""
    if workspace_bytes is None:
        workspace_bytes = workspace.numel() * workspace.element_size()
    _check(
        lib().cri_fused_decode_attention_ws(
            _ptr(Q),
            _ptr(K_cache),
            _ptr(V_cache),
            _ptr(output),
            n_heads,
            n_kv_heads,
            head_dim,
            kv_len,
            float(scale),
            _ptr(workspace),
            int(workspace_bytes),
            _stream(stream),
        )
    )


def _fid(fmt):
    return FORMAT_IDS[fmt] if isinstance(fmt, str) else int(fmt)


def matmul_rmsnorm(fmt, hidden, residual, norm_weight, hidden_out, B, C, M, N, K, eps=1e-5, stream=None):
    """C = RMSNorm(hidden + residual) * dequant(B)^T with hidden + residual written to
    hidden_out (either of residual / hidden_out may be None); decode batches M <= 16."""
    _check(
        lib().cri_matmul_rmsnorm(
            _fid(fmt), _ptr(hidden), _ptr(residual), _ptr(norm_weight), _ptr(hidden_out), _ptr(B), _ptr(C),
            M, N, K, float(eps), _stream(stream),
        )
    )


def matmul_swiglu(fmt, gate, up, ld, B, C, M, N, K, stream=None):
    """C = (silu(gate) * up) * dequant(B)^T, gate/up rows ld floats apart; decode batches M <= 16."""
    _check(lib().cri_matmul_swiglu(_fid(fmt), _ptr(gate), _ptr(up), ld, _ptr(B), _ptr(C), M, N, K, _stream(stream)))


def rmsnorm_residual(input, residual, weight, output, normed, rows, n, eps=1e-5, stream=None):
    """output = input + residual; normed = RMSNorm(output) * weight (replaces cuinfer::rmsnorm_residual)."""
    _check(
        lib().cri_rmsnorm_residual(
            _ptr(input), _ptr(residual), _ptr(weight), _ptr(output), _ptr(normed), rows, n, float(eps),
            _stream(stream),
        )
    )


def silu_mul(gate, up, out, n, stream=None):
    """out = silu(gate) * up (cuinfer::silu then cuinfer::multiply, as one launch)."""
    _check(lib().cri_silu_mul(_ptr(gate), _ptr(up), _ptr(out), int(n), _stream(stream)))
