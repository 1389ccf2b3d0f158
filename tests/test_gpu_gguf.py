"""GGUF weights on the device: raw uploads bit-identical to the file, the fused
matmuls on uploaded weights against the oracle on the file's bytes, and
embedding rows from every table format bit-identical to the oracle's dequant."""
import numpy as np
import pytest

from conftest import normwise_rel_err

torch = pytest.importorskip("torch")
import cretif_amd as cri  # noqa: E402
from cretif_amd import quant  # noqa: E402
from gguf_writer import GGUFWriter, T_STR  # noqa: E402

pytestmark = pytest.mark.gpu

FMTS = ["q8_0", "q4_0", "q5_0", "q4_k", "q6_k", "fp16"]
GGML_NAME = {"q8_0": "q8_0", "q4_0": "q4_0", "q5_0": "q5_0", "q4_k": "q4_k", "q6_k": "q6_k", "fp16": "f16"}


@pytest.fixture
def model(tmp_path):
    w = GGUFWriter().add("general.architecture", T_STR, "llama")
    weights = {}
    for i, f in enumerate(FMTS):
        N, K = 40 + i, 512
        W = quant.synthetic_weights(f, N, K, seed=70 + i)
        w.add_tensor("blk.%d.w" % i, [K, N], GGML_NAME[f], W)
        weights[f] = (i, N, K, W)
    p = tmp_path / "m.gguf"
    w.write(str(p))
    return str(p), weights


def test_upload_and_matmul(orc, model):
    path, weights = model
    with cri.GGUFFile(path) as g:
        for f, (i, N, K, W) in weights.items():
            info = g.tensor(g.find_tensor("blk.%d.w" % i))
            dev = torch.full((info["byte_size"],), 0xAB, dtype=torch.uint8, device="cuda")
            g.upload(g.find_tensor("blk.%d.w" % i), dev)
            assert np.array_equal(dev.cpu().numpy(), W)
            x = quant.randn(2 * K, seed=i).reshape(2, K).astype(np.float32)
            C = torch.empty(2, N, device="cuda")
            cri.matmul(info["format"], torch.from_numpy(x).cuda(), dev, C, 2, N, K)
            torch.cuda.synchronize()
            assert normwise_rel_err(C.cpu().numpy(), orc.matmul_quant(f, x, W, N, K)) <= 1e-5


def test_upload_rejects_small_destination(model):
    path, weights = model
    with cri.GGUFFile(path) as g:
        dev = torch.empty(10, dtype=torch.uint8, device="cuda")
        with pytest.raises(cri.CretifError) as e:
            g.upload(0, dev)
        assert e.value.status == -2


@pytest.mark.parametrize("fmt", FMTS + ["fp32"])
def test_embedding_rows(orc, fmt):
    V, D = 257, 512
    if fmt == "fp32":
        table = quant.randn(V * D, seed=3).astype(np.float32)
        ref = table.reshape(V, D)
    else:
        table = quant.synthetic_weights(fmt, V, D, seed=80)
        ref = orc.dequantize(fmt, table, V * D).reshape(V, D)
    ids = np.array([0, 256, 5, 5, -3, 257, 100], np.int32)
    out = torch.full((len(ids), D), float("nan"), device="cuda")
    cri.embedding_rows(fmt, torch.from_numpy(table.view(np.uint8) if fmt != "fp32" else table).cuda(),
                       torch.from_numpy(ids).cuda(), out, len(ids), D, V)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i, t in enumerate(ids):
        expect = ref[t] if 0 <= t < V else np.zeros(D, np.float32)
        assert np.array_equal(got[i].view(np.uint32), expect.view(np.uint32)), (fmt, t)
