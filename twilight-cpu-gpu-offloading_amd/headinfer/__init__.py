"""MI355X-native sparse-decode KV path with the reference ``headinfer`` call
surface: the Quest / Twilight offload caches (quest_offload_cache,
twilight_offload_cache), the fused selection operators
(twilight_fused_quest.fused_quest_score, twilight_fused_qk.
fused_affine_int4_qk), the decode attention hook (mp.
_flash_attention_varlen_forward) and the slab bookkeeping (slab_cache).
The compute runs in hand-written gfx950 HIP kernels
(``_lib/libtwilight_hip.so``) reached through a C ABI (kernels.py); there is
no CPU compute path.
"""

__all__ = ["kernels", "slab_cache", "quest_offload_cache", "twilight_offload_cache", "twilight_fused_quest",
           "twilight_fused_qk", "mp"]
