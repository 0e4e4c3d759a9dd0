"""MI355X-native sparse-decode KV path with the reference ``headinfer`` call
surface (Quest / Twilight offload caches, fused selection kernels, sparse GQA
decode attention).  The compute runs in hand-written gfx950 HIP kernels
(``_lib/libtwilight_hip.so``) reached through a C ABI; see kernels.py.
"""

__all__ = ["kernels"]
