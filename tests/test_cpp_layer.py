"""The header-only C++ layer (include/molot_amd/attn.hpp) on the GPU: runs the
self-checking binary tests/cpp/test_attn_cpp (built by __graft_entry__.build())."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "test_attn_cpp")


@pytest.mark.gpu
def test_cpp_layer_selfcheck(gpu):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} not built (run __graft_entry__.build())")
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASSED" in r.stdout


def test_cpp_layer_binary_links():
    """CPU side: the binary exists and resolves its libraries (ldd)."""
    if not os.path.exists(BIN):
        pytest.skip("C++ self-check not built in this tree")
    out = subprocess.run(["ldd", BIN], capture_output=True, text=True).stdout
    assert "not found" not in out, out
    assert "libmolot_amd.so" in out and "liboracle.so" in out
