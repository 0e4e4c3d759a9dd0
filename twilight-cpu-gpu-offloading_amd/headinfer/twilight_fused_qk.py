"""fused_affine_int4_qk (twilight_fused_qk.py:34-55) on gfx950: FP32 QK of
per-token affine INT4 keys at candidate positions, or the dequantized keys
with materialize=True."""

from .kernels import fused_affine_int4_qk

__all__ = ["fused_affine_int4_qk"]
