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
    "matmul_ws",
    "matmul_workspace_bytes",
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
    "prefill_attention",
    "prefill_attention_workspace_bytes",
    "fused_decode_attention_noalloc",
    "decode_attention_workspace_size",
    "matmul_rmsnorm",
    "matmul_swiglu",
    "rmsnorm_residual",
    "silu_mul",
    "embedding_rows",
    "stream_read",
    "GGUFFile",
    "Decoder",
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
    -6: "CRI_ERR_FILE",
}

_MATMUL = ["cri_matmul_" + f for f in ("q8_0", "q4_0", "q5_0", "q4_k", "q6_k", "fp16")]
_DEQUANT = ["cri_dequantize_" + f for f in ("q8_0", "q4_0", "q5_0", "q6_k", "q4_k")]
ABI_SYMBOLS = (
    _MATMUL
    + ["cri_matmul", "cri_matmul_ws", "cri_matmul_workspace_bytes"]
    + _DEQUANT
    + [
        "cri_matmul_transposed_b",
        "cri_batched_matmul_gqa",
        "cri_fused_decode_attention",
        "cri_fused_decode_attention_ws",
        "cri_prefill_attention",
        "cri_prefill_attention_workspace_bytes",
        "cri_fused_decode_attention_noalloc",
        "cri_fused_decode_attention_workspace_size",
        "cri_matmul_rmsnorm",
        "cri_matmul_swiglu",
        "cri_rmsnorm_residual",
        "cri_silu_mul",
        "cri_gguf_open",
        "cri_gguf_close",
        "cri_gguf_version",
        "cri_gguf_tensor_count",
        "cri_gguf_metadata_count",
        "cri_gguf_find_tensor",
        "cri_gguf_tensor_info",
        "cri_gguf_tensor_data",
        "cri_gguf_metadata_type",
        "cri_gguf_get_u32",
        "cri_gguf_get_i32",
        "cri_gguf_get_u64",
        "cri_gguf_get_f32",
        "cri_gguf_get_string",
        "cri_gguf_get_array_length",
        "cri_gguf_model_params",
        "cri_gguf_upload",
        "cri_embedding_rows",
        "cri_decoder_create",
        "cri_decoder_destroy",
        "cri_decoder_set_layer",
        "cri_decoder_set_embedding",
        "cri_decoder_set_output",
        "cri_decoder_forward",
        "cri_decoder_prefill",
        "cri_decoder_forward_taps",
        "cri_decoder_capture",
        "cri_decoder_replay",
        "cri_decoder_set_position",
        "cri_decoder_position",
        "cri_decoder_kv_cache",
        "cri_decoder_weight_bytes",
        "cri_decoder_step_weight_bytes",
        "cri_stream_read",
        "cri_stream_read_ex",
        "cri_timestamp",
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


class _GGUFTensor(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("ggml_type", ctypes.c_int),
        ("format", ctypes.c_int),
        ("n_dims", ctypes.c_int),
        ("dims", ctypes.c_longlong * 8),
        ("n_elements", ctypes.c_longlong),
        ("byte_size", ctypes.c_longlong),
        ("data_offset", ctypes.c_longlong),
    ]


class _GGUFModel(ctypes.Structure):
    _fields_ = [("architecture", ctypes.c_char * 64)] + [
        (n, ctypes.c_uint)
        for n in ("context_length", "embedding_length", "block_count", "head_count", "head_count_kv",
                  "feed_forward_length", "rope_dimension_count", "vocab_size")
    ] + [
        ("rope_freq_base", ctypes.c_float),
        ("rms_norm_eps", ctypes.c_float),
        ("tie_word_embeddings", ctypes.c_int),
        ("missing", ctypes.c_uint),
    ]


class _DecoderConfig(ctypes.Structure):
    _fields_ = [(f, ctypes.c_int) for f in ("n_layers", "dim", "n_heads", "n_kv_heads", "head_dim", "ffn_dim",
                                            "vocab_size", "max_seq_len", "max_batch")] + [
        ("rms_norm_eps", ctypes.c_float), ("rope_theta", ctypes.c_float)]


_LAYER_MATS = ("q", "k", "v", "o", "gate", "up", "down")


class _DecoderLayer(ctypes.Structure):
    _fields_ = [("attn_norm", ctypes.c_void_p), ("ffn_norm", ctypes.c_void_p)] + [
        (n + "_format", ctypes.c_int) for n in _LAYER_MATS] + [(n, ctypes.c_void_p) for n in _LAYER_MATS]


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
    L.cri_matmul_ws.argtypes = [i32, vp, vp, vp, i32, i32, i32, vp, ctypes.c_longlong, vp]
    L.cri_matmul_ws.restype = i32
    L.cri_matmul_workspace_bytes.argtypes = [i32, i32, i32, i32]
    L.cri_matmul_workspace_bytes.restype = ctypes.c_longlong
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
    L.cri_prefill_attention.argtypes = [vp, i32, vp, vp, vp, i32, i32, i32, i32, i32, ctypes.c_float, vp,
                                        ctypes.c_longlong, vp]
    L.cri_prefill_attention.restype = i32
    L.cri_prefill_attention_workspace_bytes.argtypes = [i32, i32, i32, i32, i32]
    L.cri_prefill_attention_workspace_bytes.restype = ctypes.c_longlong
    L.cri_fused_decode_attention_noalloc.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, ctypes.c_float, vp]
    L.cri_fused_decode_attention_noalloc.restype = i32
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
    L.cri_embedding_rows.argtypes = [i32, vp, vp, vp, i32, i32, i32, vp]
    L.cri_stream_read.argtypes = [vp, ctypes.c_longlong, vp, vp]
    L.cri_stream_read_ex.argtypes = [vp, ctypes.c_longlong, vp, i32, i32, vp]
    L.cri_stream_read_ex.restype = i32
    L.cri_timestamp.argtypes = [vp, vp]
    L.cri_timestamp.restype = i32
    L.cri_embedding_rows.restype = i32
    ll = ctypes.c_longlong
    L.cri_gguf_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(vp)]
    L.cri_gguf_open.restype = i32
    L.cri_gguf_close.argtypes = [vp]
    L.cri_gguf_close.restype = None
    L.cri_gguf_version.argtypes = [vp]
    L.cri_gguf_version.restype = i32
    for n in ("cri_gguf_tensor_count", "cri_gguf_metadata_count"):
        getattr(L, n).argtypes = [vp]
        getattr(L, n).restype = ll
    L.cri_gguf_find_tensor.argtypes = [vp, ctypes.c_char_p]
    L.cri_gguf_find_tensor.restype = i32
    L.cri_gguf_tensor_info.argtypes = [vp, i32, ctypes.POINTER(_GGUFTensor)]
    L.cri_gguf_tensor_info.restype = i32
    L.cri_gguf_tensor_data.argtypes = [vp, i32]
    L.cri_gguf_tensor_data.restype = vp
    L.cri_gguf_metadata_type.argtypes = [vp, ctypes.c_char_p]
    L.cri_gguf_metadata_type.restype = i32
    for n, t in (("u32", ctypes.c_uint), ("i32", ctypes.c_int), ("u64", ctypes.c_ulonglong), ("f32", ctypes.c_float),
                 ("string", ctypes.c_char_p)):
        f = getattr(L, "cri_gguf_get_" + n)
        f.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(t)]
        f.restype = i32
    L.cri_gguf_get_array_length.argtypes = [vp, ctypes.c_char_p]
    L.cri_gguf_get_array_length.restype = ll
    L.cri_gguf_model_params.argtypes = [vp, ctypes.POINTER(_GGUFModel)]
    L.cri_gguf_model_params.restype = i32
    L.cri_gguf_upload.argtypes = [vp, i32, vp, ll, vp]
    L.cri_gguf_upload.restype = i32
    L.cri_decoder_create.argtypes = [ctypes.POINTER(_DecoderConfig), ctypes.POINTER(vp)]
    L.cri_decoder_create.restype = i32
    L.cri_decoder_destroy.argtypes = [vp]
    L.cri_decoder_destroy.restype = None
    L.cri_decoder_set_layer.argtypes = [vp, i32, ctypes.POINTER(_DecoderLayer)]
    L.cri_decoder_set_layer.restype = i32
    L.cri_decoder_set_embedding.argtypes = [vp, i32, vp]
    L.cri_decoder_set_embedding.restype = i32
    L.cri_decoder_set_output.argtypes = [vp, vp, i32, vp]
    L.cri_decoder_set_output.restype = i32
    for n in ("cri_decoder_forward", "cri_decoder_capture", "cri_decoder_prefill"):
        getattr(L, n).argtypes = [vp, vp, i32, vp, vp, vp]
        getattr(L, n).restype = i32
    L.cri_decoder_forward_taps.argtypes = [vp, vp, i32, vp, vp, vp, vp]
    L.cri_decoder_forward_taps.restype = i32
    L.cri_decoder_replay.argtypes = [vp, vp]
    L.cri_decoder_replay.restype = i32
    L.cri_decoder_set_position.argtypes = [vp, i32, vp]
    L.cri_decoder_set_position.restype = i32
    L.cri_decoder_position.argtypes = [vp]
    L.cri_decoder_position.restype = i32
    L.cri_decoder_kv_cache.argtypes = [vp, i32, ctypes.POINTER(vp), ctypes.POINTER(vp)]
    L.cri_decoder_kv_cache.restype = i32
    L.cri_decoder_weight_bytes.argtypes = [vp]
    L.cri_decoder_weight_bytes.restype = ll
    L.cri_decoder_step_weight_bytes.argtypes = [vp, i32]
    L.cri_decoder_step_weight_bytes.restype = ll
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


def matmul_workspace_bytes(fmt, M, N, K):
    """Workspace bytes matmul_ws uses for this shape (0 when none)."""
    fid = FORMAT_IDS[fmt] if isinstance(fmt, str) else int(fmt)
    n = lib().cri_matmul_workspace_bytes(fid, M, N, K)
    if n < 0:
        _check(int(n))
    return int(n)


def matmul_ws(fmt, A, B, C, M, N, K, workspace, workspace_bytes=None, stream=None):
    """matmul with a caller workspace: 2..16-row products add their K-split partial sums in a
    fixed order (the same bits on every call).  No counterpart in the reference."""
    fid = FORMAT_IDS[fmt] if isinstance(fmt, str) else int(fmt)
    if workspace_bytes is None:
        workspace_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check(lib().cri_matmul_ws(fid, _ptr(A), _ptr(B), _ptr(C), M, N, K, _ptr(workspace), workspace_bytes,
                               _stream(stream)))


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


def prefill_attention_workspace_bytes(M, n_heads, n_kv_heads, head_dim, kv_len):
    return int(lib().cri_prefill_attention_workspace_bytes(M, n_heads, n_kv_heads, head_dim, kv_len))


def prefill_attention(Q, ldq, K_cache, V_cache, output, M, n_heads, n_kv_heads, head_dim, pos, scale,
                      workspace=None, workspace_bytes=None, stream=None):
    """Prompt attention, the reference's prefill flow (ref:src/attention.cu:809-871): M rotated
    query rows (ldq floats apart) at positions pos .. pos + M - 1 over the [kv_len, n_kv_heads,
    head_dim] caches, row m attending to positions <= pos + m.  workspace: a device tensor (one is
    allocated when None)."""
    need = prefill_attention_workspace_bytes(M, n_heads, n_kv_heads, head_dim, pos + M)
    if workspace is None:
        import torch

        workspace = torch.empty((need + 3) // 4, dtype=torch.float32, device="cuda")
    if workspace_bytes is None:
        workspace_bytes = workspace.numel() * workspace.element_size()
    _check(lib().cri_prefill_attention(_ptr(Q), ldq, _ptr(K_cache), _ptr(V_cache), _ptr(output), M, n_heads,
                                       n_kv_heads, head_dim, pos, float(scale), _ptr(workspace), int(workspace_bytes),
                                       _stream(stream)))


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


def fused_decode_attention_noalloc(Q, K_cache, V_cache, output, n_heads, n_kv_heads, head_dim, kv_len, scale,
                                   stream=None):
    """cri_fused_decode_attention_noalloc: the split form with its records in the library's
    static per-GPU scratch (no workspace, no allocation; calls on one GPU must not overlap)."""
    _check(lib().cri_fused_decode_attention_noalloc(_ptr(Q), _ptr(K_cache), _ptr(V_cache), _ptr(output), n_heads,
                                                    n_kv_heads, head_dim, kv_len, float(scale), _stream(stream)))


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


def embedding_rows(fmt, table, ids, out, n_ids, dim, vocab, stream=None):
    """out[i] = dequant(table row ids[i]) (zero rows for ids outside [0, vocab)); fmt may be 'fp32'."""
    fid = 6 if fmt == "fp32" else _fid(fmt)
    _check(lib().cri_embedding_rows(fid, _ptr(table), _ptr(ids), _ptr(out), n_ids, dim, vocab, _stream(stream)))


def stream_read(src, n_bytes, sink, stream=None):
    """Read n_bytes (a multiple of 16) at src once with 16-byte loads: the achievable streaming-read
    bandwidth (a measurement aid).  sink is one device word, written only if the XOR of the words one
    thread reads (four 16-byte chunks, 4096 bytes apart) equals 0x9E3779B9."""
    _check(lib().cri_stream_read(_ptr(src), n_bytes, _ptr(sink), _stream(stream)))


def timestamp(dst, stream=None):
    """cri_timestamp: the GPU's 100 MHz clock into dst (a device int64 tensor element or address)."""
    _check(lib().cri_timestamp(_ptr(dst), _stream(stream)))


def stream_read_ex(src, n_bytes, sink, loads_per_thread=4, grid_blocks=0, stream=None):
    """cri_stream_read_ex: the streaming-read probe with its launch shape as parameters."""
    _check(lib().cri_stream_read_ex(_ptr(src), int(n_bytes), _ptr(sink), loads_per_thread, grid_blocks,
                                    _stream(stream)))


_MODEL_FIELDS = ("context_length", "embedding_length", "block_count", "head_count", "head_count_kv",
                 "feed_forward_length", "rope_dimension_count", "vocab_size")


class GGUFFile:
    """A GGUF file opened through cri_gguf_* (the reader of cuinfer::GGUFParser).
    Metadata getters raise CretifError on a missing key or a type mismatch."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        _check(lib().cri_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            lib().cri_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def version(self):
        return lib().cri_gguf_version(self._h)

    @property
    def tensor_count(self):
        return lib().cri_gguf_tensor_count(self._h)

    @property
    def metadata_count(self):
        return lib().cri_gguf_metadata_count(self._h)

    def tensor(self, index):
        t = _GGUFTensor()
        _check(lib().cri_gguf_tensor_info(self._h, index, ctypes.byref(t)))
        return {
            "name": t.name.decode(),
            "ggml_type": t.ggml_type,
            "format": t.format,
            "dims": [t.dims[i] for i in range(t.n_dims)],
            "n_elements": t.n_elements,
            "byte_size": t.byte_size,
            "data_offset": t.data_offset,
        }

    def tensors(self):
        return [self.tensor(i) for i in range(self.tensor_count)]

    def find_tensor(self, name):
        i = lib().cri_gguf_find_tensor(self._h, name.encode())
        return None if i < 0 else i

    def tensor_bytes(self, index):
        """A copy of the tensor's raw bytes (host)."""
        import numpy as np

        info = self.tensor(index)
        p = lib().cri_gguf_tensor_data(self._h, index)
        return np.frombuffer(ctypes.string_at(p, info["byte_size"]), dtype=np.uint8).copy()

    def metadata_type(self, key):
        return lib().cri_gguf_metadata_type(self._h, key.encode())

    def _get(self, kind, ctype, key):
        v = ctype()
        _check(getattr(lib(), "cri_gguf_get_" + kind)(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def get_u32(self, key):
        return self._get("u32", ctypes.c_uint, key)

    def get_i32(self, key):
        return self._get("i32", ctypes.c_int, key)

    def get_u64(self, key):
        return self._get("u64", ctypes.c_ulonglong, key)

    def get_f32(self, key):
        return self._get("f32", ctypes.c_float, key)

    def get_string(self, key):
        return self._get("string", ctypes.c_char_p, key).decode()

    def array_length(self, key):
        n = lib().cri_gguf_get_array_length(self._h, key.encode())
        if n < 0:
            _check(int(n))
        return n

    def model_params(self):
        m = _GGUFModel()
        _check(lib().cri_gguf_model_params(self._h, ctypes.byref(m)))
        out = {"architecture": m.architecture.decode(), "rope_freq_base": m.rope_freq_base,
               "rms_norm_eps": m.rms_norm_eps, "tie_word_embeddings": bool(m.tie_word_embeddings)}
        for i, f in enumerate(_MODEL_FIELDS):
            out[f] = None if m.missing >> i & 1 else getattr(m, f)
        return out

    def upload(self, index, dst, dst_bytes=None, stream=None):
        """Copy the tensor's raw bytes to a device buffer (returns when done)."""
        if dst_bytes is None:
            dst_bytes = dst.numel() * dst.element_size()
        _check(lib().cri_gguf_upload(self._h, index, _ptr(dst), int(dst_bytes), _stream(stream)))


def _host_or_device_ptr(x):
    """Address of a host numpy array (C-contiguous) or of a device tensor / int address."""
    try:
        import numpy as np
    except ImportError:  # pragma: no cover
        np = None
    if np is not None and isinstance(x, np.ndarray):
        if not x.flags["C_CONTIGUOUS"]:
            raise ValueError("host arrays must be C-contiguous")
        return x.ctypes.data
    return _ptr(x)


_FMT_OR_FP32 = dict(FORMAT_IDS, fp32=6)


class Decoder:
    """The decode step (cri_decoder_*, C++ cuinfer::DecodeStep): the reference's quantized
    forward pass (ref:src/model.cu:831-1039) over buffers allocated at construction.
    Weights are copied in from host numpy arrays or device tensors; forward / replay run
    M tokens at the current position and advance it."""

    def __init__(self, n_layers, dim, n_heads, n_kv_heads, head_dim, ffn_dim, vocab_size, max_seq_len,
                 max_batch=16, rms_norm_eps=1e-5, rope_theta=10000.0):
        c = _DecoderConfig(n_layers, dim, n_heads, n_kv_heads, head_dim, ffn_dim, vocab_size, max_seq_len, max_batch,
                           rms_norm_eps, rope_theta)
        h = ctypes.c_void_p()
        _check(lib().cri_decoder_create(ctypes.byref(c), ctypes.byref(h)))
        self._h = h
        self.config = {f: getattr(c, f) for f, _ in _DecoderConfig._fields_}
        self._keep = []  # host arrays stay alive until their copies are done (copies are synchronous)

    def close(self):
        if getattr(self, "_h", None):
            lib().cri_decoder_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_layer(self, layer, attn_norm, ffn_norm, **mats):
        """mats: q, k, v, o, gate, up, down, each (fmt, data) with data [N, K] GGUF blocks."""
        w = _DecoderLayer()
        w.attn_norm = _host_or_device_ptr(attn_norm)
        w.ffn_norm = _host_or_device_ptr(ffn_norm)
        for n in _LAYER_MATS:
            fmt, data = mats[n]
            setattr(w, n + "_format", FORMAT_IDS[fmt])
            setattr(w, n, _host_or_device_ptr(data))
        _check(lib().cri_decoder_set_layer(self._h, layer, ctypes.byref(w)))

    def set_embedding(self, fmt, table):
        _check(lib().cri_decoder_set_embedding(self._h, _FMT_OR_FP32[fmt], _host_or_device_ptr(table)))

    def set_output(self, output_norm, lm_head=None):
        """lm_head: (fmt, data), or None to tie the head to the token table."""
        fmt, data = (-1, None) if lm_head is None else (_FMT_OR_FP32[lm_head[0]], _host_or_device_ptr(lm_head[1]))
        _check(lib().cri_decoder_set_output(self._h, _host_or_device_ptr(output_norm), fmt, data))

    def forward(self, token_ids, M, logits, next_ids=None, stream=None):
        _check(lib().cri_decoder_forward(self._h, _ptr(token_ids), M, _ptr(logits), _ptr(next_ids),
                                         _stream(stream)))

    def prefill(self, token_ids, M, logits, next_id=None, stream=None):
        """A prompt as the reference's generate() consumes it: every layer on the M tokens, the
        LM head and argmax for the last token only (logits: device fp32 [vocab])."""
        _check(lib().cri_decoder_prefill(self._h, _ptr(token_ids), M, _ptr(logits), _ptr(next_id),
                                         _stream(stream)))

    def forward_taps(self, token_ids, M, logits, hidden_taps, next_ids=None, stream=None):
        """forward() that also writes the residual stream entering each layer and the final
        norm into hidden_taps (device fp32 [n_layers + 1, M, dim])."""
        _check(lib().cri_decoder_forward_taps(self._h, _ptr(token_ids), M, _ptr(logits), _ptr(next_ids),
                                              _ptr(hidden_taps), _stream(stream)))

    def capture(self, token_ids, M, logits, next_ids=None, stream=None):
        _check(lib().cri_decoder_capture(self._h, _ptr(token_ids), M, _ptr(logits), _ptr(next_ids),
                                         _stream(stream)))

    def replay(self, stream=None):
        _check(lib().cri_decoder_replay(self._h, _stream(stream)))

    @property
    def position(self):
        return lib().cri_decoder_position(self._h)

    def set_position(self, pos, stream=None):
        _check(lib().cri_decoder_set_position(self._h, pos, _stream(stream)))

    def kv_cache(self, layer):
        """(k, v) device addresses of the layer's [max_seq_len, n_kv_heads, head_dim] caches."""
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        _check(lib().cri_decoder_kv_cache(self._h, layer, ctypes.byref(k), ctypes.byref(v)))
        return k.value, v.value

    @property
    def weight_bytes(self):
        return int(lib().cri_decoder_weight_bytes(self._h))

    def step_weight_bytes(self, M):
        """Weight bytes one step of M tokens reads (M token-table rows, not the whole table)."""
        return int(lib().cri_decoder_step_weight_bytes(self._h, M))
