"""Write the golden fixtures of the reference's pure-CPU helpers.

Run in a container that holds the reference tree (it is read, never copied):
    python tests/golden/make_fixtures.py [reference_root]

Imports only twilight_offload_cache's CPU functions -- affine_int4_pack,
affine_int4_dequantize, matched_budget_counts, matched_budget_counts_tensor
(source/headinfer/headinfer/twilight_offload_cache.py:25-130) -- and saves
their inputs and outputs as .npz data (no pickles) next to this script.  The
tests compare the oracle and the GPU kernels against these files; nothing at
test time imports the reference.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def main() -> None:
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    sys.path.insert(0, str(root / "source" / "headinfer"))
    from headinfer.twilight_offload_cache import (  # noqa: E402
        affine_int4_dequantize,
        affine_int4_pack,
        matched_budget_counts,
        matched_budget_counts_tensor,
    )

    # ---- INT4 pack / dequantize, per key dtype ----
    arrays = {}
    for name, dtype in (("f32", torch.float32), ("f16", torch.float16), ("bf16", torch.bfloat16)):
        g = torch.Generator().manual_seed(7)
        keys = (torch.randn(17, 128, generator=g) * 2.0).to(dtype)
        keys[3] = 0.5                        # constant row: scale clamps
        keys[5] *= 1e-3                      # tiny range
        keys[6, ::2] = -0.0                  # signed zeros
        keys[9] = torch.linspace(-4, 4, 128).to(dtype)  # codes hit every rounding boundary
        keys[11, :64] = 1e4 if dtype != torch.float16 else 6e4  # wide range
        packed, scale, minimum = affine_int4_pack(keys)
        restored = affine_int4_dequantize(packed, scale, minimum)
        bits = torch.int16 if dtype != torch.float32 else torch.int32
        arrays[f"{name}_keys"] = keys.view(bits).numpy()
        arrays[f"{name}_packed"] = packed.numpy()
        arrays[f"{name}_scale"] = scale.view(bits).numpy()
        arrays[f"{name}_minimum"] = minimum.view(bits).numpy()
        arrays[f"{name}_restored"] = restored.numpy()
    np.savez(HERE / "int4_pack.npz", **arrays)

    # ---- matched budget counts ----
    cases = []
    rng = np.random.default_rng(11)
    fixed = [([10, 20, 30], 33, [50, 50, 50]), ([100, 1, 1], 12, [4, 20, 20]), ([7, 7, 7], 20, [24] * 3),
             ([3, 8, 5], 11, [20] * 3), ([1], 1, [1]), ([5, 5, 5, 5], 4, [9] * 4), ([1, 2, 3, 4, 5, 6, 7], 49, [49] * 7)]
    for _ in range(40):
        heads = int(rng.integers(1, 9))
        cap = int(rng.integers(4, 5000))
        desired = [int(v) for v in rng.integers(1, cap + 1, heads)]
        target = int(rng.integers(heads, cap + 1))
        fixed.append((desired, target, [cap] * heads))
    for desired, target, caps in fixed:
        counts = matched_budget_counts(desired, target, caps)
        entry = {"desired": desired, "target": target, "capacities": caps, "counts": counts}
        if len(set(caps)) == 1 and target <= caps[0]:
            entry["counts_tensor"] = matched_budget_counts_tensor(
                torch.tensor([desired]), target, caps[0]).tolist()[0]
        cases.append(entry)
    (HERE / "matched_budget_counts.json").write_text(json.dumps(cases, indent=1) + "\n")
    print(f"wrote {HERE / 'int4_pack.npz'} and {HERE / 'matched_budget_counts.json'} ({len(cases)} cases)")


if __name__ == "__main__":
    main()
