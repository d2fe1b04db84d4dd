"""Builds and runs tests/cpp/test_kudnn_api.cpp against libkudnn.so (the KuDNN-compatible C++ API).

The CPU run covers descriptors, validation and the exception types of the reference gtests' negative cases;
the GPU run adds numeric cases that pass host buffers to Run, as the reference tests do."""
import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "tests" / "cpp" / "test_kudnn_api.cpp"
LIB = ROOT / "kudnn_amd" / "lib"
ORACLE = ROOT / "oracle"


@pytest.fixture(scope="module")
def binary(tmp_path_factory):
    for so in (LIB / "libkudnn.so", LIB / "libkudnn_hip.so", ORACLE / "liboracle.so"):
        assert so.exists(), f"{so} missing: run __graft_entry__.build()"
    out = tmp_path_factory.mktemp("cpp") / "test_kudnn_api"
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", str(ROOT / "include"), "-I", str(ORACLE), str(SRC),
           "-L", str(LIB), "-lkudnn", "-lkudnn_hip", "-L", str(ORACLE), "-loracle",
           f"-Wl,-rpath,{LIB}", f"-Wl,-rpath,{ORACLE}", "-o", str(out)]
    subprocess.run(cmd, check=True)
    return out


def test_cpp_api_host_cases(binary):
    r = subprocess.run([str(binary)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 failed" in r.stdout


@pytest.mark.gpu
def test_cpp_api_numeric_host_buffers(binary):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    r = subprocess.run([str(binary), "--gpu"], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
