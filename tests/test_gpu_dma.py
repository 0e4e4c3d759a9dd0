"""The side-stream DMA pipeline (the reference's post-selection pipeline,
twilight_offload_cache.py:2053-2455): chunked CPU gather from a pinned slab +
H2D copies on a second stream.  Rows must arrive bit-exact (index_select is
the oracle), each chunk's consumer must see its chunk's rows, and the Twilight
cache's post_selection_pipeline path must give the same K/V layout, bit for
bit, as the zero-copy gather kernel."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from helpers import randn, same_bits
from test_gpu_cache import H, _Model, _twilight_cache  # noqa: F401

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_pipeline_rows_bit_exact_and_ordered(dev):
    from headinfer.dma_pipeline import HostGatherPipeline, union_rows

    _say("[dma pipeline] rows")
    rows_total, D = 20000, 128
    k = randn((rows_total, D), "bf16", seed=301).pin_memory()
    v = randn((rows_total, D), "bf16", seed=302).pin_memory()
    rng = np.random.default_rng(303)
    sizes = [0, 1, 4000, 1777, 4096, 3, 2500]
    pipe = HostGatherPipeline(dev, D, torch.bfloat16, max_rows=4096)
    dk = torch.zeros((sum(sizes), D), dtype=torch.bfloat16, device=dev)
    dv = torch.zeros_like(dk)
    seen = torch.zeros((sum(sizes), D), dtype=torch.bfloat16, device=dev)
    chunks, offs, all_rows = [], [0], []
    for n in sizes:
        r = rng.integers(0, rows_total, size=n).astype(np.int64)
        if n > 10:
            r[:10] = np.arange(500, 510)          # a contiguous run
        a = offs[-1]
        chunks.append((r, dk[a:a + n], dv[a:a + n]))
        offs.append(a + n)
        all_rows.append(r)

    def consume(c: int) -> None:               # runs behind chunk c's copy on the compute stream
        a, b = offs[c], offs[c + 1]
        seen[a:b].copy_(dk[a:b])

    for _ in range(2):                          # the second run reuses both staging buffers
        dk.zero_()
        seen.zero_()
        pipe.run(k.view(-1, D), v.view(-1, D), chunks, on_chunk=consume)
        torch.cuda.synchronize()
        want = torch.from_numpy(np.concatenate(all_rows))
        assert same_bits(dk, k.index_select(0, want)) and same_bits(dv, v.index_select(0, want))
        assert same_bits(seen, dk)
    with pytest.raises(ValueError):
        pipe.run(k.view(-1, D), v.view(-1, D), [(np.zeros(5000, np.int64), dk[:5000], dv[:5000])])
    pos = union_rows(np.array([0, 3]), length=200, sink=4, recent=16, block_size=8)
    assert pos.tolist() == list(range(4)) + list(range(4, 12)) + list(range(28, 36)) + list(range(185, 200))


@pytest.mark.parametrize("per_chunk", [1, 3])
def test_twilight_post_selection_pipeline_matches_zero_copy(H, dev, per_chunk):
    """update_layer_gqa_group_ragged with post_selection_pipeline (host slab)
    == the zero-copy gather, bit for bit, over two decode steps of 2 layers."""
    layers, G, R, D, T = 2, 4, 4, 128, 2000
    E = layers * G
    _say(f"[dma twilight] groups per chunk {per_chunk}")
    common = dict(E=E, T=T, D=D, R=R, dtype="bf16", residency="host", mode="dynamic", candidate_token_budget=256,
                  top_p=0.9, layer_batched_selection=True, gqa_groupwise_execution=True, gpu_compact_gqa_union=True,
                  cpu_flat_gather=True, direct_attention_layout=True, gather_h2d_chunks=2)
    zc = _twilight_cache(H, dev, **common)
    dma = _twilight_cache(H, dev, post_selection_pipeline=True, post_selection_groups_per_chunk=per_chunk, **common)
    model = _Model(E, T, D, "bf16", seed=311, scale=2.0)
    model.prefill(zc, dev)
    model.prefill(dma, dev)
    g = torch.Generator().manual_seed(312)
    for step in range(2):
        for layer in range(layers):
            entries = list(range(layer * G, layer * G + G))
            qs = [(torch.randn(1, R, 1, D, generator=g) * 2).to(torch.bfloat16).to(dev) for _ in entries]
            new = [model.new_token(D) for _ in entries]
            kw = dict(key_states=[k[None, None, None].to(dev) for k, _ in new],
                      value_states=[v[None, None, None].to(dev) for _, v in new], queries=qs, entries=entries)
            a = zc.update_layer_gqa_group_ragged(**kw)
            b = dma.update_layer_gqa_group_ragged(**kw)
            torch.cuda.synchronize()
            n = int(a[2][-1])
            assert a[3] == b[3] and a[4] == b[4]
            assert torch.equal(a[2].cpu(), b[2].cpu())
            assert same_bits(a[0][:n], b[0][:n]) and same_bits(a[1][:n], b[1][:n]), (step, layer)
            for e, (nk, nv) in zip(entries, new):
                model.append(e, nk, nv)
    assert dma._dma is not None and dma._dma.rows_moved > 0
