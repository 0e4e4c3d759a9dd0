"""fused_quest_score (twilight_fused_quest.py:35-46): the Quest upper-bound
page score on gfx950, bit-exact with the reference's order (per lane l of 32
accumulating channels l, l+32, l+64, l+96, then an adjacent-pair tree; no
fused multiply-add)."""

from .kernels import fused_quest_score

__all__ = ["fused_quest_score"]
