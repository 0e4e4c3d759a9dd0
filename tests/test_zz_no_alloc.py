"""tw_quest_select_static (the entry point that allocates nothing) against
tw_quest_select on the same inputs: scores, page ids, union plan and row plan
bit for bit, on calls in a row (the second smaller, so it runs on the first
call's leftover scratch; the third with more groups, so more arrival counters
than the first call zeroed), then replayed from a captured graph with eager
work between the replays."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import oracle
from helpers import randn, to_bits

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _inputs(dev, G, R, P, D, dtype, seed):
    q = randn((G, R, D), "f32", seed=seed)
    a = randn((G, P, D), dtype, seed=seed + 1)
    b = randn((G, P, D), dtype, seed=seed + 2)
    lo = torch.minimum(a.float(), b.float()).to(a.dtype)
    hi = torch.maximum(a.float(), b.float()).to(a.dtype)
    return q.to(dev), lo.to(dev), hi.to(dev)


def _outputs(dev, G, R, P, k, length):
    width = min(P, R * k)
    return dict(scores=torch.full((G, R, P), -1.0, device=dev),
                sel=torch.full((G, R, k), -1, dtype=torch.int32, device=dev),
                pp=torch.full((G, width), -1, dtype=torch.int32, device=dev),
                pm=torch.zeros((G, width), dtype=torch.uint8, device=dev),
                pc=torch.zeros((G,), dtype=torch.int32, device=dev),
                rows=torch.full((G, length + 1), -1, dtype=torch.int32, device=dev),
                rm=torch.zeros((G, length + 1), dtype=torch.uint8, device=dev),
                rc=torch.zeros((G,), dtype=torch.int32, device=dev))


def _call_static(q, lo, hi, k, o, sink, recent, bs, length, append):
    from headinfer import _native, kernels

    G, R, D = q.shape
    P = lo.shape[1]
    with torch.cuda.device(q.device):
        rc = _native.hip().tw_quest_select_static(
            q.data_ptr(), lo.data_ptr(), hi.data_ptr(), kernels._dt(lo), G, R, P, D, lo.stride(0), k,
            o["scores"].data_ptr(), o["sel"].data_ptr(), o["pp"].data_ptr(), o["pm"].data_ptr(), o["pc"].data_ptr(),
            o["pp"].stride(0), o["rows"].data_ptr(), o["rm"].data_ptr(), o["rc"].data_ptr(), o["rows"].stride(0),
            sink, recent, bs, length, append, torch.cuda.current_stream().cuda_stream)
    _native.check(rc, "quest_select_static")


def _call_workspace(q, lo, hi, k, o, sink, recent, bs, length, append):
    from headinfer import kernels

    kernels.quest_select(q, lo, hi, k, scores=o["scores"], sel_pages=o["sel"], plan_pages=o["pp"],
                         plan_masks=o["pm"], plan_counts=o["pc"], rows=o["rows"], row_masks=o["rm"],
                         row_counts=o["rc"], sink=sink, recent=recent, block_size=bs, length=length,
                         append_position=append)


def _same(a: dict, b: dict) -> bool:
    ok = True
    for name in a:
        x, y = a[name].cpu(), b[name].cpu()
        if x.dtype == torch.float32:
            x, y = x.view(torch.int32), y.view(torch.int32)
        ok &= bool(torch.equal(x, y))
    return ok


CASES = [  # (G, R, D, dtype, length, k): the 32K layer, then a smaller one on the leftover scratch,
    # then one with more groups than the first call's zeroed arrival counters cover
    (8, 4, 128, "f16", 32768, 128),
    (3, 2, 64, "bf16", 3000, 20),
    (96, 2, 64, "f16", 3000, 20),
]


def test_static_scratch_matches_workspace_entry_point(dev):
    from headinfer import _native

    assert _native.hip().tw_quest_select_static_capacity() == 16 << 20
    sink, recent, bs = 64, 256, 16
    for i, (G, R, D, dtype, length, k) in enumerate(CASES):
        _say(f"[no-alloc] call {i}: G={G} R={R} D={D} {dtype} L={length} k={k}")
        sink_end, recent_start, eligible = oracle.selection_window(length, sink, recent)
        P = eligible // bs
        q, lo, hi = _inputs(dev, G, R, P, D, dtype, seed=10 * i + 1)
        a, b = _outputs(dev, G, R, P, k, length), _outputs(dev, G, R, P, k, length)
        _call_static(q, lo, hi, k, a, sink, recent, bs, length, length)
        _call_workspace(q, lo, hi, k, b, sink, recent, bs, length, length)
        torch.cuda.synchronize()
        assert _same(a, b), i
        # and the page ids are the oracle's
        sc = oracle.quest_score(q[:1].cpu().numpy(), to_bits(lo[:1]), to_bits(hi[:1]), dtype)[0]
        assert np.array_equal(a["sel"][0].cpu().numpy(), oracle.topk_sorted(sc, k)), i


def test_static_scratch_graph_replays(dev):
    G, R, D, dtype, length, k = 4, 4, 128, "bf16", 8192, 64
    sink, recent, bs = 64, 256, 16
    _say("[no-alloc] graph replays")
    P = oracle.selection_window(length, sink, recent)[2] // bs
    q, lo, hi = _inputs(dev, G, R, P, D, dtype, seed=77)
    ref = _outputs(dev, G, R, P, k, length)
    _call_workspace(q, lo, hi, k, ref, sink, recent, bs, length, -1)
    got = _outputs(dev, G, R, P, k, length)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            _call_static(q, lo, hi, k, got, sink, recent, bs, length, -1)
    torch.cuda.current_stream().wait_stream(s)
    init = _outputs(dev, G, R, P, k, length)
    for rep in range(3):
        for name, t in got.items():   # the fill the reference call started from
            t.copy_(init[name])
        # eager work on the same scratch between replays
        other = _outputs(dev, 2, 2, 300, 10, 5120)
        q2, lo2, hi2 = _inputs(dev, 2, 2, 300, 64, "f16", seed=100 + rep)
        _call_static(q2, lo2, hi2, 10, other, sink, recent, bs, 5120, -1)
        graph.replay()
        torch.cuda.synchronize()
        assert _same(got, ref), rep
