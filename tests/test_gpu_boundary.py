"""GPU checks of boundary contracts: the gather's destination bounds, the
cache's deferred gather-error report, and scratch workspaces that outgrow
their buffer while a captured graph still holds the old address."""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
import torch

import oracle
from helpers import randn, same_bits

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def K():
    from headinfer import kernels

    return kernels


def test_gather_rows_destination_bounds(K, dev):
    """Destination rows outside the destination buffer are skipped and
    flagged (like bad source rows); without dst_rows the row count must fit."""
    _say("[gather dst bounds]")
    D = 128
    k = randn((100, D), "f16", seed=1).to(dev)
    v = randn((100, D), "f16", seed=2).to(dev)
    dk = torch.zeros((4, D), dtype=torch.float16, device=dev)
    dv = torch.zeros_like(dk)
    flag = torch.zeros((), dtype=torch.int32, device=dev)
    src = torch.tensor([3, 4, 5, 6, 7], device=dev)
    dst = torch.tensor([0, 4, -1, 3, 1000], device=dev)
    K.gather_rows(k, v, src, dk, dv, dst, error_flag=flag)
    torch.cuda.synchronize()
    assert int(flag) == 1
    assert same_bits(dk[0], k[3].cpu()) and same_bits(dk[3], k[6].cpu())
    assert (dk[[1, 2]].float() == 0).all()
    with pytest.raises(ValueError, match="do not fit"):
        K.gather_rows(k, v, torch.arange(5, device=dev), dk, dv)


def test_cache_reports_gather_error_at_synchronize(dev):
    from headinfer.quest_offload_cache import QuestTopKOffloadedCache

    cache = QuestTopKOffloadedCache(num_cache_entries=1, max_cache_len=64, head_dim=8, num_query_heads_per_kv=1,
                                    dtype=torch.float16, device=dev, kv_residency="hbm")
    cache.synchronize()
    cache._gather_error.fill_(1)      # as a gather kernel that met a bad row leaves it
    with pytest.raises(RuntimeError, match="outside the slab"):
        cache.synchronize()
    cache.synchronize()               # reported once, then cleared


def test_graph_replay_after_workspace_regrowth(K, dev):
    """A graph captured over the shared attention workspace replays
    correctly after a larger call replaced that workspace: the outgrown
    buffer stays allocated and its counters stay zero."""
    _say("[workspace regrowth]")
    G, R, D, L = 4, 4, 128, 2048
    q = randn((G, R, D), "f16", seed=3).to(dev)
    kc = randn((G, L, D), "f16", seed=4).to(dev)
    vc = randn((G, L, D), "f16", seed=5).to(dev)
    n_rows = 600
    gen = torch.Generator().manual_seed(6)
    rows = torch.stack([torch.randperm(L, generator=gen)[:n_rows].sort().values for _ in range(G)]).to(torch.int32)
    counts = torch.full((G,), n_rows, dtype=torch.int32)
    rows_d, counts_d = rows.to(dev), counts.to(dev)
    K.WORKSPACE._buffers.pop((torch.device(dev), "decode_attention"), None)
    out = torch.empty_like(q)
    K.decode_attention_rows(q, kc, vc, rows_d, counts_d, n_rows, out=out)       # sizes the workspace
    eager = out.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            K.decode_attention_rows(q, kc, vc, rows_d, counts_d, n_rows, out=out)
    torch.cuda.current_stream().wait_stream(s)
    small = K.WORKSPACE._buffers[(torch.device(dev), "decode_attention")].numel()
    # a much larger call replaces the workspace
    big_rows = torch.arange(L, dtype=torch.int32, device=dev).repeat(G, 1)
    big = K.decode_attention_rows(q, kc, vc, big_rows, torch.full((G,), L, dtype=torch.int32, device=dev), L)
    assert K.WORKSPACE._buffers[(torch.device(dev), "decode_attention")].numel() > small
    scribble = torch.full((small // 4 + 1024,), -1, dtype=torch.int32, device=dev)  # reuse of freed memory shows up
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert same_bits(out, eager)
    ref = np.zeros((G, R, D))
    for g in range(G):
        r = rows[g].long()
        ref[g] = oracle.decode_attention(q[g].float().cpu().numpy(), kc[g, r].float().cpu().numpy(),
                                         vc[g, r].float().cpu().numpy(), 1.0 / math.sqrt(D))
    assert np.abs(out.float().cpu().numpy() - ref).max() < 2e-3 + 1e-2 * np.abs(ref).max()
    del big, scribble
