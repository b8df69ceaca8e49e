"""dwarf_amd -- MI355X-native (gfx950) DSQG fixed-offset sparse attention.

Forward, backward and a ring-buffer decode step are HIP kernels in libdsqg_hip.so (C ABI:
include/dsqg.h), exposed as torch custom ops (``dwarf::dsqg_fwd``, ``dwarf::dsqg_bwd``,
``dwarf::dsqg_decode``) and wrapped with the reference's call signatures; so is the block's
interference pool (``dwarf::pool_gate_fwd`` / ``_bwd``).
"""

from .offsets import ALL_OFFSETS, OFFSETS_V3, OFFSETS_J46, OFFSETS_J47
from .api import (dsqg_attention, dsqg_attention_qkv, dsqg_attention_v2, dsqg_attention_v3,
                  dsqg_attention_backend, dsqg_attention_with_lse, dsqg_decode_step,
                  causal_mean_pool_gate, DSQGRingCache)
from .modules import DSQGAttentionV3, DSQGAttentionQW, DSQGAttentionN_Fused, DSQGBlock, FFN
from .generation import CondMTransformer, FullAttentionBlock, FullCausalAttention

__all__ = ["ALL_OFFSETS", "OFFSETS_V3", "OFFSETS_J46", "OFFSETS_J47", "dsqg_attention",
           "dsqg_attention_qkv",
           "dsqg_attention_v2", "dsqg_attention_v3", "dsqg_attention_backend",
           "dsqg_attention_with_lse", "dsqg_decode_step", "causal_mean_pool_gate",
           "DSQGRingCache", "DSQGAttentionV3", "DSQGAttentionQW", "DSQGAttentionN_Fused",
           "DSQGBlock", "FFN", "CondMTransformer", "FullAttentionBlock", "FullCausalAttention"]
