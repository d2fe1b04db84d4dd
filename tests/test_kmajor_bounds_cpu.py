"""CPU check of the ping-pong kernel's K-major weight copy addresses (kudnn_amd/csrc/kmajor_copy.h).

tests/cpp/test_kmajor_bounds.cpp walks every copy of every tile with the kernel's own address helpers and the raw
buffer range rule: no byte past the weight's last byte is read, every in-matrix element is read at its own address,
and the whole-tile form would overrun on the edge tiles (so the check can fail)."""
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_kmajor_copy_bounds(tmp_path):
    exe = tmp_path / "test_kmajor_bounds"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", str(ROOT / "kudnn_amd" / "csrc"),
                    str(ROOT / "tests" / "cpp" / "test_kmajor_bounds.cpp"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 failures" in r.stdout
