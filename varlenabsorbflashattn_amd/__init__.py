"""MI355X (gfx950) packed varlen FlashAttention and absorbed target attention.

Drop-in replacements for the reference packages' public APIs:

* ``triton_fa_varlen_v2``: :func:`packed_varlen_attn`, :func:`set_validate_cu_seqlens`
* ``triton_target_attn_absorb``: :func:`packed_target_attn`,
  :func:`target_attn_inner`, :func:`prepare_target_attn_indices`

All compute runs in the in-tree HIP library ``libvafa.so`` (C ABI in
``include/vafa.h``); it is loaded on the first call.
"""
from .varlen import packed_varlen_attn, set_validate_cu_seqlens
from .absorb import packed_target_attn, prepare_target_attn_indices, target_attn_inner

__all__ = [
    "packed_varlen_attn",
    "set_validate_cu_seqlens",
    "packed_target_attn",
    "prepare_target_attn_indices",
    "target_attn_inner",
]
__version__ = "0.1.0"
