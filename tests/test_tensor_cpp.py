"""cuinfer::Tensor (the drop-in for the reference's Tensor) compiled into a host
program against libcretif.so: shape, view, reshape and move errors on the CPU,
the reference's device-tensor test list (ref:tests/test_tensor.cu:12-230) on
the GPU."""
import os
import shutil
import subprocess

import pytest

import cretif_amd  # noqa: F401  (the library must be built)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ not found")
    out = str(tmp_path_factory.mktemp("cpp") / "tensor_check")
    libdir = os.path.join(ROOT, "cretif_amd")
    cmd = [cxx, "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"), "-I",
           "/opt/rocm/include", os.path.join(ROOT, "tests", "cpp", "tensor_check.cpp"), "-L", libdir, "-lcretif",
           "-Wl,-rpath," + libdir, "-L", "/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib", "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return out


def test_tensor_errors_cpu(checker):
    r = subprocess.run([checker, "cpu"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr


@pytest.mark.gpu
def test_tensor_reference_list_gpu(checker):
    r = subprocess.run([checker, "gpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr
