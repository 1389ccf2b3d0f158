"""The C ABI library loads, exports every function include/cri.h declares, and
rejects bad arguments before touching the GPU (so this runs without one)."""
import ctypes
import os
import re

import pytest

import cretif_amd as cri

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    names = []
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if h.endswith(".h"):
            text = open(os.path.join(ROOT, "include", h)).read()
            names += re.findall(r"^\s*(?:int|long long|void|const void\*|const char\*)\s+(cri_\w+)\s*\(", text, re.M)
    return names


def test_header_declares_abi():
    names = header_functions()
    assert len(names) >= 18
    assert set(names) == set(cri.ABI_SYMBOLS)


def test_library_exports_every_symbol():
    L = ctypes.CDLL(cri.library_path)
    for name in header_functions():
        assert hasattr(L, name), name


def test_block_tables():
    L = cri.lib()
    assert [L.cri_block_bytes(i) for i in range(6)] == [34, 18, 22, 144, 210, 2]
    assert [L.cri_block_elems(i) for i in range(6)] == [32, 32, 32, 256, 256, 1]
    assert L.cri_block_bytes(99) == 0
    assert L.cri_version() >= 100


FAKE = 1 << 20  # never dereferenced: every case below fails validation first


@pytest.mark.parametrize(
    "fn,K,status",
    [
        ("matmul_q8_0", 48, -2),
        ("matmul_q4_0", 33, -2),
        ("matmul_q5_0", 16, -2),
        ("matmul_q4_k", 512 + 32, -2),
        ("matmul_q6_k", 128, -2),
        ("matmul_fp16", 40, -2),
    ],
)
def test_bad_k_rejected(fn, K, status):
    with pytest.raises(cri.CretifError) as e:
        getattr(cri, fn)(FAKE, FAKE, FAKE, 1, 8, K, stream=0)
    assert e.value.status == status
    assert "multiple" in str(e.value)


def test_negative_dims_and_nulls():
    with pytest.raises(cri.CretifError) as e:
        cri.matmul_q8_0(FAKE, FAKE, FAKE, -1, 8, 32, stream=0)
    assert e.value.status == -1
    with pytest.raises(cri.CretifError) as e:
        cri.matmul_q4_k(0, FAKE, FAKE, 1, 8, 256, stream=0)
    assert e.value.status == -1
    with pytest.raises(cri.CretifError) as e:
        cri.dequantize_q6_k(FAKE, FAKE, -3, stream=0)
    assert e.value.status == -1


def test_misaligned_rejected():
    with pytest.raises(cri.CretifError) as e:
        cri.matmul_q8_0(FAKE + 2, FAKE, FAKE, 1, 8, 32, stream=0)
    assert e.value.status == -3
    with pytest.raises(cri.CretifError) as e:
        cri.matmul_fp16(FAKE, FAKE + 1, FAKE, 1, 8, 32, stream=0)
    assert e.value.status == -3


def test_empty_problems_are_noops():
    # M == 0 or N == 0 or n_blocks == 0: nothing to launch, success
    cri.matmul_q8_0(0, 0, 0, 0, 8, 32, stream=0)
    cri.matmul_q4_k(0, 0, 0, 4, 0, 256, stream=0)
    cri.dequantize_q4_k(0, 0, 0, stream=0)
    cri.batched_matmul_gqa(0, 0, 0, 0, 8, 1, 64, 64, stream=0)


def test_unknown_format():
    with pytest.raises(cri.CretifError) as e:
        cri.matmul(17, FAKE, FAKE, FAKE, 1, 8, 32, stream=0)
    assert e.value.status == -5


def test_gqa_head_ratio():
    with pytest.raises(cri.CretifError) as e:
        cri.batched_matmul_gqa(FAKE, FAKE, FAKE, 6, 4, 1, 64, 64, stream=0)
    assert e.value.status == -2
    with pytest.raises(cri.CretifError) as e:
        cri.batched_matmul_gqa(FAKE, FAKE, FAKE, 4, 0, 1, 64, 64, stream=0)
    assert e.value.status == -2


def test_cpu_tensor_rejected():
    torch = pytest.importorskip("torch")
    A = torch.zeros(1, 32)
    with pytest.raises(ValueError):
        cri.matmul_q8_0(A, A, A, 1, 1, 32, stream=0)


def test_decode_attention_validation():
    f = cri.fused_decode_attention
    for args, status in [
        ((32, 8, 64, 0), -2),      # empty cache (the reference would return NaN)
        ((6, 4, 64, 10), -2),      # n_heads not a multiple of n_kv_heads
        ((4, 0, 64, 10), -2),
        ((4, 4, 257, 10), -2),     # head_dim above the kernel's limit
        ((4, 4, -1, 10), -1),
        ((4, 4, 64, -5), -1),
    ]:
        with pytest.raises(cri.CretifError) as e:
            f(FAKE, FAKE, FAKE, FAKE, *args, 0.125, stream=0)
        assert e.value.status == status, args
    with pytest.raises(cri.CretifError) as e:
        f(0, FAKE, FAKE, FAKE, 4, 4, 64, 10, 0.125, stream=0)
    assert e.value.status == -1
    with pytest.raises(cri.CretifError) as e:
        f(FAKE, FAKE + 2, FAKE, FAKE, 4, 4, 64, 10, 0.125, stream=0)
    assert e.value.status == -3
    f(0, 0, 0, 0, 0, 8, 64, 10, 0.125, stream=0)  # no heads: nothing to do


def test_decode_attention_ws_validation():
    assert cri.decode_attention_workspace_size(32, 8, 64, 2048) > 0
    assert cri.decode_attention_workspace_size(0, 8, 64, 2048) == 0
    with pytest.raises(cri.CretifError) as e:
        cri.decode_attention_workspace_size(6, 4, 64, 10)
    assert e.value.status == -2
    f = cri.fused_decode_attention_ws
    with pytest.raises(cri.CretifError) as e:   # argument errors are reported as in the workspace-free form
        f(FAKE, FAKE, FAKE, FAKE, 32, 8, 64, 0, 0.125, FAKE, 1 << 20, stream=0)
    assert e.value.status == -2 and "cri_fused_decode_attention_ws" in str(e.value)
    with pytest.raises(cri.CretifError) as e:
        f(FAKE, FAKE, FAKE, FAKE, 32, 8, 64, 100, 0.125, 0, 1 << 20, stream=0)
    assert e.value.status == -1
    with pytest.raises(cri.CretifError) as e:
        f(FAKE, FAKE, FAKE, FAKE, 32, 8, 64, 100, 0.125, FAKE + 4, 1 << 20, stream=0)
    assert e.value.status == -3
    with pytest.raises(cri.CretifError) as e:   # not even one record per head
        f(FAKE, FAKE, FAKE, FAKE, 32, 8, 64, 100, 0.125, FAKE, 100, stream=0)
    assert e.value.status == -2


def test_fused_prologue_validation():
    with pytest.raises(cri.CretifError) as e:
        cri.matmul_rmsnorm("q4_k", FAKE, None, FAKE, None, FAKE, FAKE, 1, 8, 0, stream=0)
    assert e.value.status == -2
    with pytest.raises(cri.CretifError) as e:
        cri.matmul_rmsnorm("q4_k", FAKE, None, 0, None, FAKE, FAKE, 1, 8, 256, stream=0)
    assert e.value.status == -1
    with pytest.raises(cri.CretifError) as e:   # hidden_out overlapping hidden
        cri.matmul_rmsnorm("q4_k", FAKE, None, FAKE, FAKE + 64, FAKE, FAKE, 1, 8, 256, stream=0)
    assert e.value.status == -1
    with pytest.raises(cri.CretifError) as e:
        cri.matmul_rmsnorm("q4_k", FAKE, None, FAKE, None, FAKE, FAKE, 17, 8, 256, stream=0)
    assert e.value.status == -5
    with pytest.raises(cri.CretifError) as e:
        cri.matmul_swiglu("q4_k", FAKE, FAKE, 128, FAKE, FAKE, 1, 8, 256, stream=0)
    assert e.value.status == -2
    with pytest.raises(cri.CretifError) as e:
        cri.matmul_swiglu("q8_0", FAKE, FAKE, 64, FAKE, FAKE, 1, 8, 48, stream=0)
    assert e.value.status == -2
    with pytest.raises(cri.CretifError) as e:
        cri.rmsnorm_residual(FAKE, None, FAKE, FAKE, FAKE, 2, 0, stream=0)
    assert e.value.status == -2
    with pytest.raises(cri.CretifError) as e:
        cri.silu_mul(FAKE, FAKE, FAKE + 2, 10, stream=0)
    assert e.value.status == -3
    cri.silu_mul(0, 0, 0, 0, stream=0)
    cri.matmul_swiglu("q4_k", 0, 0, 0, 0, 0, 0, 8, 256, stream=0)


def test_stream_read_validation():
    with pytest.raises(cri.CretifError) as e:
        cri.stream_read(FAKE, 24, FAKE, stream=0)  # not a multiple of 16
    assert e.value.status == -1
    with pytest.raises(cri.CretifError) as e:
        cri.stream_read(FAKE + 8, 64, FAKE, stream=0)
    assert e.value.status == -3
    with pytest.raises(cri.CretifError) as e:
        cri.stream_read(0, 64, FAKE, stream=0)
    assert e.value.status == -1
    cri.stream_read(0, 0, 0, stream=0)
