"""cri_fused_decode_attention_noalloc (no reference counterpart; for callers that
cannot allocate) through the C ABI against cri_fused_decode_attention_ws, the
entry point whose kernels it shares: bit-identical outputs on two calls in a
row, the second with a smaller input, plus its argument errors."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
import cretif_amd as cri  # noqa: E402

pytestmark = pytest.mark.gpu


def case(H, Hkv, D, T, seed):
    rng = np.random.default_rng(seed)
    q = torch.from_numpy(rng.standard_normal(H * D).astype(np.float32)).cuda()
    k = torch.from_numpy(rng.standard_normal(T * Hkv * D).astype(np.float32)).cuda()
    v = torch.from_numpy(rng.standard_normal(T * Hkv * D).astype(np.float32)).cuda()
    return q, k, v


def run_ws(q, k, v, H, Hkv, D, T, scale):
    out = torch.full((H * D,), float("nan"), device="cuda")
    ws = torch.empty(max(4, cri.decode_attention_workspace_size(H, Hkv, D, T) // 4), device="cuda")
    cri.fused_decode_attention_ws(q, k, v, out, H, Hkv, D, T, scale, ws)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def run_noalloc(q, k, v, H, Hkv, D, T, scale):
    out = torch.full((H * D,), float("nan"), device="cuda")
    cri.fused_decode_attention_noalloc(q, k, v, out, H, Hkv, D, T, scale)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_noalloc_matches_ws_twice_second_smaller():
    # a Llama-3.2-1B decode shape, then a smaller one: the second call reuses the scratch the
    # first one filled (more chunks, more heads) and must not read any of it
    for (H, Hkv, D, T, seed) in ((32, 8, 64, 2048, 1), (8, 2, 32, 77, 2)):
        q, k, v = case(H, Hkv, D, T, seed)
        a = run_noalloc(q, k, v, H, Hkv, D, T, 0.125)
        b = run_ws(q, k, v, H, Hkv, D, T, 0.125)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (H, Hkv, D, T)


def test_noalloc_head_dim_128_and_long_cache():
    # head_dim 128 and 8192 positions: the records still fit, the chunking equals the ws form's
    H, Hkv, D, T = 32, 8, 128, 8192
    q, k, v = case(H, Hkv, D, T, 3)
    assert np.array_equal(run_noalloc(q, k, v, H, Hkv, D, T, 0.08).view(np.uint32),
                          run_ws(q, k, v, H, Hkv, D, T, 0.08).view(np.uint32))


def test_noalloc_rejects_what_does_not_fit():
    q, k, v = case(4, 2, 6, 10, 4)
    with pytest.raises(cri.CretifError) as e:  # head_dim % 4 != 0: no split kernel
        run_noalloc(q, k, v, 4, 2, 6, 10, 0.1)
    assert e.value.status == -5
    # 2048 heads x (128 + 4) floats: one record per head is past the 1 MiB scratch
    H, D = 2048, 128
    q = torch.zeros(H * D, device="cuda")
    kv = torch.zeros(4 * 1 * D, device="cuda")
    with pytest.raises(cri.CretifError) as e:
        cri.fused_decode_attention_noalloc(q, kv, kv, torch.empty(H * D, device="cuda"), H, 1, D, 4, 0.1)
    assert e.value.status == -2 and "static scratch" in str(e.value)
