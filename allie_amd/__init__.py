"""allie_amd: MI355X (gfx950) engine for Allie's batched policy/value inference.

Host side in Python over a C-ABI library of hand-written HIP kernels
(``liballie_amd.so``, built by ``allie_amd.build``).
"""
from . import config, vocab  # noqa: F401

__all__ = ["config", "vocab"]
