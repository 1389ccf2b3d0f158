"""The reference-shaped C++ API (include/cuinfer/) compiled and run as a host
program against libcretif.so: GGUFParser semantics on the CPU; the tied
quantized LM head, a Q4_K weight and the embedding rows on the GPU, checked
against the oracle."""
import os
import shutil
import subprocess

import numpy as np
import pytest

import cretif_amd as cri
from cretif_amd import quant
from gguf_writer import GGUFWriter, T_STR, T_U32

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
K, VOCAB, FF = 512, 300, 96


def model_file(tmp_path):
    w = GGUFWriter().add("general.architecture", T_STR, "llama").add("llama.embedding_length", T_U32, K)
    emb = quant.synthetic_weights("q6_k", VOCAB, K, seed=5)
    up = quant.synthetic_weights("q4_k", FF, K, seed=6)
    w.add_tensor("token_embd.weight", [K, VOCAB], "q6_k", emb)
    w.add_tensor("blk.0.ffn_up.weight", [K, FF], "q4_k", up)
    p = tmp_path / "tiny.gguf"
    w.write(str(p))
    return str(p), emb, up


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ not found")
    out = str(tmp_path_factory.mktemp("cpp") / "gguf_api_check")
    libdir = os.path.join(ROOT, "cretif_amd")
    cmd = [cxx, "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"), "-I",
           "/opt/rocm/include", os.path.join(ROOT, "tests", "cpp", "gguf_api_check.cpp"), "-L", libdir, "-lcretif",
           "-Wl,-rpath," + libdir, "-L", "/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib", "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return out


def test_cpp_parser_api(checker, tmp_path):
    path, _, _ = model_file(tmp_path)
    r = subprocess.run([checker, path], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr


@pytest.mark.gpu
def test_cpp_tied_lm_head_and_embedding(checker, tmp_path, orc):
    path, emb, up = model_file(tmp_path)
    x = quant.randn(K, seed=9).astype(np.float32)
    (tmp_path / "x.bin").write_bytes(x.tobytes())
    ids = [0, 7, VOCAB - 1, -1, VOCAB]
    out = tmp_path / "out.bin"
    r = subprocess.run([checker, path, "--gpu", str(out), str(tmp_path / "x.bin"), ",".join(map(str, ids))],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "ok gpu" in r.stdout, r.stdout + r.stderr
    got = np.fromfile(str(out), dtype=np.float32)
    y, u, rows = got[:VOCAB], got[VOCAB:VOCAB + FF], got[VOCAB + FF:].reshape(len(ids), K)
    from conftest import normwise_rel_err

    assert normwise_rel_err(y, orc.matmul_quant("q6_k", x.reshape(1, K), emb, VOCAB, K)[0]) <= 1e-5
    assert normwise_rel_err(u, orc.matmul_quant("q4_k", x.reshape(1, K), up, FF, K)[0]) <= 1e-5
    table = orc.dequantize("q6_k", emb, VOCAB * K).reshape(VOCAB, K)
    for i, t in enumerate(ids):
        ref = table[t] if 0 <= t < VOCAB else np.zeros(K, np.float32)
        assert np.array_equal(rows[i].view(np.uint32), ref.view(np.uint32))
