"""MI355X (gfx950) paged-attention path for the lucciola-rs Qwen2 engine.

The product is the C-ABI library lib/liblucattn.so (include/luc_attn.h) and the
gfx950 code objects it loads.  This package binds it for Python callers:

* ``library`` -- ctypes binding of every C-ABI entry point, over torch tensors
  (torch provides device memory and streams);
* ``engine``  -- the reference engine's host-side API for this path
  (RopeCache, KVCache, apply_rope, apply_flash_decoding), written over the
  binding, plus batched forms.

There is no fallback: if the library is missing or fails to load, every call
raises.
"""
from .library import LucAttn, LucError, lib_dir  # noqa: F401
from .engine import (  # noqa: F401
    RopeCache,
    KVCache,
    apply_rope,
    apply_flash_decoding,
    decode_step,
)
