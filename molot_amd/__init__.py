"""molot_amd: MI355X-native fused RoPE + GQA decode attention.

The product is the C-ABI library libmolot_amd.so (HIP kernels for gfx950,
declared in include/molot_amd/attn_hip.h) plus the header-only C++ layer
include/molot_amd/attn.hpp.  This package is the Python host binding used by
tests and bench.py; it needs the built library and a GPU for any compute call.
"""
from .lib import KV_BF16, KV_F32, EXPORTS, LIB_PATH, MolotHipError, load  # noqa: F401

__version__ = "0.1"
