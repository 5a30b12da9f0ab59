"""The header-only C++ layer (include/molot_amd/attn.hpp, paged_kv.hpp) on the
GPU: runs the self-checking binaries tests/cpp/test_attn_cpp and
tests/cpp/test_paged_kv (built by __graft_entry__.build())."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "test_attn_cpp")
BIN_PAGED = os.path.join(HERE, "cpp", "test_paged_kv")


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


@pytest.mark.gpu
def test_paged_kv_manager_selfcheck(gpu):
    """Continuous batching through PagedKVCache: prefill, batched decode over
    two layers, a freed sequence's blocks reused, a full pool's error."""
    if not os.path.exists(BIN_PAGED):
        pytest.fail(f"{BIN_PAGED} not built (run __graft_entry__.build())")
    r = subprocess.run([BIN_PAGED], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASSED" in r.stdout


def test_paged_kv_binary_links():
    if not os.path.exists(BIN_PAGED):
        pytest.skip("paged-KV self-check not built in this tree")
    out = subprocess.run(["ldd", BIN_PAGED], capture_output=True, text=True).stdout
    assert "not found" not in out, out
    assert "libmolot_amd.so" in out and "liboracle.so" in out
