"""Build recipes for the native parts of molot_amd (run on the CPU host).

``build_all()`` compiles, in-tree:
  molot_amd/libmolot_amd.so   HIP kernels + C ABI (hipcc, gfx950): the drop-in
  molot_amd/libmolot_probe.so bench-only streaming probes (include/molot_amd/probe.h)
  tests/cpp/test_attn_cpp      C++ self-check of the header-only C++ layer
  tests/cpp/test_paged_kv      C++ self-check of the paged-KV manager
                              (include/molot_amd/attn.hpp), linked to the above
                              and to the oracle (its checker)
  tests/cpp/host_io_time       time of the C++ drop-in's decode call with host
                              vectors against device ones (bench.py's host_io)
The oracle (oracle/Makefile) is test infrastructure and is built by
``__graft_entry__.build()`` next to these, never by the product path.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "molot_amd")
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(PKG, "libmolot_amd.so")
PROBE_LIB = os.path.join(PKG, "libmolot_probe.so")
CPP_TEST = os.path.join(ROOT, "tests", "cpp", "test_attn_cpp")
ARCH = os.environ.get("MOLOT_OFFLOAD_ARCH", "gfx950")

# Packed-FP32 VALU forms are kept out of the generated code: -packed-fp32-ops.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # single-lane atomics only: no wave-level scan around them (it would wait
    # for an atomic's return right where it is issued)
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build molot_amd)")


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_library() -> str:
    tmp = LIB + ".tmp"
    _run([_hipcc(), *HIP_FLAGS, "-shared", f"-I{INCLUDE}", os.path.join(CSRC, "attn_decode.hip"),
          "-o", tmp])
    os.replace(tmp, LIB)
    return LIB


def build_probe_library() -> str:
    tmp = PROBE_LIB + ".tmp"
    _run([_hipcc(), *HIP_FLAGS, "-shared", f"-I{INCLUDE}", os.path.join(CSRC, "probe.hip"),
          "-o", tmp])
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def build_cpp_test(name: str = "test_attn_cpp") -> str:
    src = os.path.join(ROOT, "tests", "cpp", name + ".cpp")
    out = os.path.join(ROOT, "tests", "cpp", name)
    oracle_inc = os.path.join(ROOT, "oracle")
    tmp = out + ".tmp"
    # rpaths relative to the binary, so the tree can move (the GPU box copies it)
    _run([_hipcc(), *HIP_FLAGS, f"-I{INCLUDE}", f"-I{oracle_inc}", src, "-o", tmp,
          f"-L{PKG}", "-lmolot_amd", f"-L{os.path.join(ROOT, 'oracle')}", "-loracle",
          "-Wl,-rpath,$ORIGIN/../../molot_amd", "-Wl,-rpath,$ORIGIN/../../oracle"])
    os.replace(tmp, out)
    return out


CPP_TESTS = ("test_attn_cpp", "test_paged_kv", "host_io_time")


def build_all() -> None:
    build_library()
    build_probe_library()
    for name in CPP_TESTS:
        if os.path.exists(os.path.join(ROOT, "tests", "cpp", name + ".cpp")):
            build_cpp_test(name)


if __name__ == "__main__":
    build_all()
    sys.exit(0)
