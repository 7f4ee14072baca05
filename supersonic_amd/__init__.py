"""MI355X (gfx950) full-attention hot path of SuperSonic's Qwen3.5/3.6 layers.

The compute lives in ``libsupersonic_attn.so`` (hand-written HIP, built in-tree
by ``supersonic_amd.build``); ``kernel_ffi`` binds its C ABI.
"""
from . import kernel_ffi  # noqa: F401

__all__ = ["kernel_ffi"]
