"""The C ABI boundary, checked on the CPU (no compute call needs a GPU here).

- libmolot_amd.so loads and exports every function include/molot_amd/attn_hip.h
  declares (and the Python binding knows each one), and nothing else of this
  library's namespace: the measurement probes (include/molot_amd/probe.h)
  live in the bench-only libmolot_probe.so;
- host-only functions (status strings, version, the RoPE table) work;
- argument validation rejects bad shapes with status codes before anything
  touches the device.
"""
import ctypes
import glob
import os
import re
import subprocess

import numpy as np
import pytest

import oracle
from molot_amd import lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include", "molot_amd")
HEADERS = sorted(glob.glob(os.path.join(INC, "*.h")))
ABI_HEADER = os.path.join(INC, "attn_hip.h")
PROBE_HEADER = os.path.join(INC, "probe.h")


def declared_functions(headers=(ABI_HEADER,)):
    names = set()
    for h in headers:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names.update(re.findall(r"\b(molot_\w+)\s*\(", text))
    return sorted(names)


def exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True,
                         capture_output=True, text=True).stdout
    return set(re.findall(r" T (\w+)", out))


def test_header_declarations_match_binding():
    assert set(HEADERS) == {ABI_HEADER, PROBE_HEADER}, HEADERS
    decl = declared_functions()
    assert decl == sorted(L.EXPORTS), set(decl) ^ set(L.EXPORTS)
    probes = declared_functions((PROBE_HEADER,))
    assert probes == L.PROBE_EXPORTS, set(probes) ^ set(L.PROBE_EXPORTS)


def test_library_exports_every_declared_symbol():
    ours = {f for f in exported(L.LIB_PATH) if f.startswith("molot_")}
    assert ours == set(declared_functions()), ours ^ set(declared_functions())
    probes = {f for f in exported(L.PROBE_LIB_PATH) if f.startswith("molot_")}
    assert probes == set(L.PROBE_EXPORTS), probes


def test_library_loads_and_binds():
    lib = L.load()
    for name in L.EXPORTS:
        assert callable(getattr(lib, name))
    assert lib.molot_hip_version().decode().startswith("molot_amd")


def test_status_strings():
    lib = L.load()
    assert lib.molot_hip_strerror(0) == b"ok"
    assert b"invalid" in lib.molot_hip_strerror(L.EINVAL)
    assert b"unsupported" in lib.molot_hip_strerror(L.ENOTSUP)
    assert b"full" in lib.molot_hip_strerror(L.ENOSPC)
    assert b"4 MiB scratch" in lib.molot_hip_strerror(L.E2BIG)


@pytest.mark.parametrize("base,d", [(500000.0, 128), (10000.0, 256), (10000.0, 64)])
def test_host_inv_freq_matches_oracle(base, d):
    out = (ctypes.c_float * (d // 2))()
    L.load().molot_rope_inv_freq(base, d, out)
    got = np.frombuffer(out, dtype=np.float32)
    assert np.array_equal(got, oracle.rope_inv_freq(base, d))


def _p(v=0x1000):  # a dummy non-null pointer: never dereferenced on these paths
    return ctypes.c_void_p(v)


def test_validation_before_launch():
    lib = L.load()
    s = ctypes.c_void_p(0)
    # nq not a multiple of nkv
    assert lib.molot_hip_attn_decode_gqa_cache(_p(), _p(), _p(), _p(), 6, 4, 10, 128, 0.1, 9, 0,
                                               0, s) == L.EINVAL
    # unknown kv dtype
    assert lib.molot_hip_attn_decode_gqa_cache(_p(), _p(), _p(), _p(), 8, 4, 10, 128, 0.1, 9, 0,
                                               7, s) == L.EINVAL
    # head dims without kernels: decode and prefill take any even d up to 512
    for d in (97, 514, 0, 1024):
        assert lib.molot_hip_attn_decode_gqa_cache(_p(), _p(), _p(), _p(), 8, 4, 10, d, 0.1, 9,
                                                   0, 0, s) == L.ENOTSUP
    # prefill: any even d up to 512 on fp32 and bf16 caches; Q8 any multiple of 4
    for d, kvd in ((514, 0), (514, L.KV_BF16), (90, L.KV_Q8), (34, L.KV_Q8), (7, 0)):
        assert lib.molot_hip_attn_prefill_gqa(_p(), _p(), _p(), _p(), 8, 2, 4, 10, d, 0.1, 6, 0,
                                              kvd, s) == L.ENOTSUP
        assert lib.molot_hip_prefill_step(_p(), _p(), _p(), _p(), _p(), _p(), 8, 2, d, 4, 6, 6,
                                          None, None, 0, 1e-6, _p(), 0.1, 0, kvd,
                                          s) == L.ENOTSUP
    assert lib.molot_hip_attn_decode_gqa_cache(_p(), _p(), _p(), _p(), 8, 2, 10, 98, 0.1, 9, 0,
                                               L.KV_Q8, s) == L.ENOTSUP
    # null output
    assert lib.molot_hip_attn_decode_strided(_p(), _p(), _p(), None, 8, 4, 10, 128, 512, 128,
                                             0.1, 9, 0, 0, s) == L.EINVAL
    # misaligned K (16-byte vector loads)
    assert lib.molot_hip_attn_decode_strided(_p(), _p(0x1004), _p(), _p(), 8, 4, 10, 128, 512,
                                             128, 0.1, 9, 0, 0, s) == L.EINVAL
    # odd head dim for RoPE, negative slot
    assert lib.molot_hip_rope_apply(_p(), 4, 127, 3, _p(), s) == L.EINVAL
    assert lib.molot_hip_rope_append(_p(), _p(), _p(), _p(), _p(), 8, 4, 128, -1, 3, _p(), 0,
                                     s) == L.EINVAL
    # paged: page size must be a power of two; lengths must fit the table
    assert lib.molot_hip_attn_decode_paged(_p(), _p(), _p(), _p(), _p(), _p(), None, 2, 4, 40, 8,
                                           4, 128, 12, 0.1, 0, 0, s) == L.EINVAL
    assert lib.molot_hip_attn_decode_paged(_p(), _p(), _p(), _p(), _p(), _p(), None, 2, 4, 100, 8,
                                           4, 128, 16, 0.1, 0, 0, s) == L.EINVAL
    nch, ch = ctypes.c_int(), ctypes.c_int()
    assert lib.molot_hip_last_plan(None, ctypes.byref(ch)) == L.EINVAL


def test_python_layer_checks_sizes_without_gpu():
    """Host-side size checks run before any pointer is passed."""
    import torch
    from molot_amd import attn

    cpu = torch.zeros(10)
    with pytest.raises(ValueError, match="device tensor"):
        attn.attn_decode_gqa_cache(cpu, cpu, cpu, cpu, 1, 1, 10, 128, 0.1, 9, 0)


def test_q8_layout_sizes_match_oracle():
    lib = L.load()
    for nkv, d, page in [(8, 128, 16), (2, 64, 16), (1, 64, 4), (3, 128, 8), (16, 64, 32)]:
        assert lib.molot_hip_q8_row_bytes(nkv, d) == oracle.q8_row_bytes(nkv, d)
        assert lib.molot_hip_q8_block_bytes(nkv, d, page) == oracle.q8_block_bytes(nkv, d, page)
    # 1024 codes + 8 scales (32 bytes, already 16-byte aligned); 3 heads: 12 -> 16 bytes
    assert lib.molot_hip_q8_row_bytes(8, 128) == 1056
    assert lib.molot_hip_q8_row_bytes(3, 128) == 3 * 128 + 16
    assert lib.molot_hip_q8_block_bytes(8, 128, 16) == 8 * 16 * 128 + 4 * 8 * 16
    assert lib.molot_hip_q8_row_bytes(0, 128) == 0


def test_q8_validation_before_launch():
    lib = L.load()
    s = ctypes.c_void_p(0)
    Q8 = L.KV_Q8
    # Q8 caches: any multiple of 4 up to 512 (a token's fp32 scales follow its codes)
    for d in (90, 34, 516, 2):
        assert lib.molot_hip_attn_decode_gqa_cache(_p(), _p(), _p(), _p(), 8, 2, 10, d, 0.1, 9,
                                                   0, Q8, s) == L.ENOTSUP
    # element strides instead of the token-major Q8 byte layout
    assert lib.molot_hip_attn_decode_strided(_p(), _p(), _p(), _p(), 8, 2, 10, 128, 256, 128,
                                             0.1, 9, 0, Q8, s) == L.EINVAL
    # the head-major entry points take no Q8 cache
    assert lib.molot_hip_attn_decode_gqa(_p(), _p(), _p(), _p(), 8, 2, 10, 64, 0.1, Q8,
                                         s) == L.EINVAL
    # paged Q8 blocks stay 16-byte aligned only when nkv * page is a multiple of 4
    assert lib.molot_hip_attn_decode_paged(_p(), _p(), _p(), _p(), _p(), _p(), None, 1, 4, 4, 8,
                                           1, 64, 2, 0.1, 0, Q8, s) == L.EINVAL
    assert lib.molot_hip_attn_prefill_gqa(_p(), _p(), _p(), _p(), 8, 2, 4, 10, 190, 0.1, 6, 0,
                                          Q8, s) == L.ENOTSUP  # Q8 prefill: multiples of 4
    # the RoPE/append entries write only rows the attention entries read back
    assert lib.molot_hip_rope_append(_p(), _p(), _p(), _p(), _p(), 8, 2, 190, 5, 5, _p(), Q8,
                                     s) == L.ENOTSUP
    assert lib.molot_hip_rope_append_paged(_p(), _p(), _p(), _p(), _p(), _p(), _p(), None, 1, 4,
                                           8, 2, 190, 16, _p(), Q8, s) == L.ENOTSUP
    assert lib.molot_hip_rope_append_paged(_p(), _p(), _p(), _p(), _p(), _p(), _p(), None, 1, 4,
                                           8, 1, 64, 2, _p(), Q8, s) == L.EINVAL
    assert lib.molot_hip_rope_append_paged(_p(), _p(), _p(), _p(), _p(), _p(), _p(), None, 1, 4,
                                           8, 2, 64, 12, _p(), 0, s) == L.EINVAL


def test_shared_kv_entries_validate_before_launch():
    lib = L.load()
    s = ctypes.c_void_p(0)
    # an empty source cache (forward.h:580 throws "shared KV empty")
    assert lib.molot_hip_decode_step_shared(_p(), _p(), _p(), _p(), 8, 2, 128, 0, 0, None, 1e-6,
                                            None, 0.1, 0, 0, s) == L.EINVAL
    # negative eps, odd head dim
    assert lib.molot_hip_decode_step_shared(_p(), _p(), _p(), _p(), 8, 2, 128, 5, 4, None, -1.0,
                                            None, 0.1, 0, 0, s) == L.EINVAL
    assert lib.molot_hip_prefill_q(_p(), 8, 127, 3, 0, None, 1e-6, _p(), s) == L.EINVAL
    # nothing to apply: no launch, success
    assert lib.molot_hip_prefill_q(_p(), 8, 128, 3, 0, None, 1e-6, None, s) == 0
    # paged prefill: N beyond the block-table row
    assert lib.molot_hip_attn_prefill_paged(_p(), _p(), _p(), _p(), _p(), 4, 16, 8, 2, 3, 65, 128,
                                            0.1, 62, 0, 0, s) == L.EINVAL
    assert lib.molot_hip_decode_step_paged_shared(_p(), _p(), _p(), _p(), _p(), _p(), None, 2, 4,
                                                  40, 8, 4, 128, 12, None, 1e-6, None, 0.1, 0, 0,
                                                  s) == L.EINVAL


def test_python_kv_dtype_codes():
    import torch
    from molot_amd import attn

    assert attn.kv_dtype_of(torch.zeros(1, dtype=torch.uint8)) == L.KV_Q8
    assert attn.kv_dtype_of(torch.zeros(1, dtype=torch.bfloat16)) == L.KV_BF16
    assert attn.kv_dtype_of(torch.zeros(1)) == L.KV_F32
    with pytest.raises(TypeError):
        attn.kv_dtype_of(torch.zeros(1, dtype=torch.float16))
