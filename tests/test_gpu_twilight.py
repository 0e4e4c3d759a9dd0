"""GPU parity of the Twilight stage-2 kernels against the CPU oracle.

One decoder layer goes through the product path exactly as the cache runs
it: prompt metadata (page min/max + INT4 keys), the stage-1 Quest B0
selection with its union plan, the INT4 QK estimate, the top-p counts, the
(matched) budgets, the token selection and the GQA token union.  Everything
is integer or fixed-order fp32, so every output is compared bit for bit with
oracle.twilight_layer (the same computation restated on the CPU).
"""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
import torch

import oracle
from helpers import TORCH_DT, randn, to_bits

pytestmark = pytest.mark.gpu


def _say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def K():
    from headinfer import kernels

    return kernels


CASES = [
    # dtype, G, R, D, L, sink, recent, bs, b0, top_p, mode, fixed_pages, temperature
    ("f16", 8, 4, 128, 4096, 64, 256, 16, 64, 0.95, "dynamic", 0, 1.0),
    ("f16", 8, 4, 128, 4096, 64, 256, 16, 64, 0.95, "matched", 16, 4.0),
    ("bf16", 2, 7, 64, 20000, 64, 256, 16, 256, 0.9, "matched", 61, 6.0),
    ("f32", 3, 8, 256, 3000, 10, 30, 8, 40, 0.5, "dynamic", 0, 2.0),
    ("bf16", 2, 4, 128, 32768, 64, 256, 16, 512, 0.95, "matched", 128, 3.0),   # N = 8192 candidates
    ("f16", 2, 4, 128, 32768, 64, 256, 16, 512, 0.99, "dynamic", 0, 0.5),
    ("f16", 4, 2, 128, 2500, 64, 256, 12, 30, 1.0, "dynamic", 0, 8.0),          # top_p = 1, page size 12
    ("bf16", 2, 1, 64, 1200, 4, 16, 4, 100, 0.3, "matched", 25, 1.0),          # one head per group
    # past 8192 candidates: 32 per thread of the 512-thread top-p block
    ("f16", 2, 4, 128, 32768, 64, 256, 16, 1024, 0.95, "dynamic", 0, 1.0),    # N = 16384, the limit
    ("bf16", 2, 4, 128, 32768, 64, 256, 16, 1024, 0.9, "matched", 300, 3.0),
    ("bf16", 3, 2, 128, 20000, 64, 256, 16, 700, 0.99, "dynamic", 0, 0.5),    # N = 11200
]


def _layer(K, dev, dtype, G, R, D, L, sink, recent, bs, b0, top_p, mode, fixed_pages, temperature, *,
           keys=None, q=None):
    sink_end, recent_start, eligible = oracle.selection_window(L, sink, recent)
    P = eligible // bs
    assert b0 <= P
    if keys is None:
        keys = randn((G, L, D), dtype, seed=L + D)
    if q is None:
        q = randn((G, R, D), "f32", seed=L + 3, scale=temperature)
    kd = keys.to(dev)
    npages = (L - sink) // bs
    pmin = torch.empty((G, npages, D), dtype=TORCH_DT[dtype], device=dev)
    pmax = torch.empty_like(pmin)
    packed = torch.empty((G, L, D // 2), dtype=torch.uint8, device=dev)
    scale = torch.empty((G, L), dtype=TORCH_DT[dtype], device=dev)
    minimum = torch.empty_like(scale)
    K.build_page_metadata(kd, sink=sink, block_size=bs, page_min=pmin, page_max=pmax, packed=packed, scale=scale,
                          minimum=minimum)
    qd = q.to(dev)
    sel = torch.empty((G, R, b0), dtype=torch.int32, device=dev)
    pw = min(P, R * b0)
    ppages = torch.empty((G, pw), dtype=torch.int32, device=dev)
    pmasks = torch.empty((G, pw), dtype=torch.uint8, device=dev)
    pcounts = torch.empty((G,), dtype=torch.int32, device=dev)
    rows = torch.full((G, L + 1), -5, dtype=torch.int32, device=dev)
    counts = torch.zeros((G,), dtype=torch.int32, device=dev)
    desired = torch.zeros((G, R), dtype=torch.int32, device=dev)
    allocated = torch.zeros((G, R), dtype=torch.int32, device=dev)
    for _ in range(2):  # repeated: the arrival counters must be left at zero
        K.quest_select(qd, pmin[:, :P], pmax[:, :P], b0, sel_pages=sel, plan_pages=ppages, plan_masks=pmasks,
                       plan_counts=pcounts)
        logits = K.twilight_qk(qd, packed, scale, minimum, ppages, pmasks, pcounts, b0, sink=sink, block_size=bs)
        K.twilight_select(logits, sel, top_p=top_p, budget_mode=mode, target_total=fixed_pages * bs * R, rows=rows,
                          row_counts=counts, desired=desired, allocated=allocated, sink=sink, recent=recent,
                          block_size=bs, length=L, append_position=L)
    torch.cuda.synchronize()
    return keys, q, sel, logits, desired, allocated, rows, counts


@pytest.mark.parametrize("dtype,G,R,D,L,sink,recent,bs,b0,top_p,mode,fixed_pages,temperature", CASES)
def test_twilight_layer_bit_exact(K, dev, dtype, G, R, D, L, sink, recent, bs, b0, top_p, mode, fixed_pages,
                                  temperature):
    _say(f"[twilight] {dtype} G={G} R={R} D={D} L={L} b0={b0} top_p={top_p} {mode}")
    keys, q, sel, logits, desired, allocated, rows, counts = _layer(
        K, dev, dtype, G, R, D, L, sink, recent, bs, b0, top_p, mode, fixed_pages, temperature)
    kb = to_bits(keys)
    qn = q.numpy()
    P = oracle.selection_window(L, sink, recent)[2] // bs
    spread = []
    for g in range(G):
        pmin, pmax, packed, sc, mn = oracle.build_page_metadata(kb[g], dtype, sink, bs)
        ref = oracle.twilight_layer(qn[g], pmin[:P], pmax[:P], packed, sc, mn, dtype, length=L, sink=sink,
                                    recent=recent, block_size=bs, b0_pages=b0, top_p=top_p, budget_mode=mode,
                                    fixed_pages=fixed_pages)
        assert np.array_equal(sel[g].cpu().numpy(), ref["pages"]), f"group {g}: B0 pages"
        got = logits[g].cpu().numpy()
        bad = np.argwhere(got.view(np.uint32) != ref["logits"].view(np.uint32))
        assert bad.size == 0, f"group {g}: {len(bad)} logits differ, first {bad[:3].tolist()}"
        assert np.array_equal(desired[g].cpu().numpy(), ref["desired"]), f"group {g}: desired"
        assert np.array_equal(allocated[g].cpu().numpy(), ref["allocated"]), f"group {g}: allocated"
        n = int(counts[g])
        assert n == len(ref["union"]) + 1, f"group {g}: union size {n - 1} vs {len(ref['union'])}"
        got_rows = rows[g, :n].cpu().numpy()
        assert np.array_equal(got_rows[:-1], ref["union"]) and got_rows[-1] == L
        if mode == "matched":
            assert int(allocated[g].sum()) == fixed_pages * bs * R
        spread.append(int(desired[g].min()))
        spread.append(int(desired[g].max()))
    _say(f"   desired range {min(spread)}..{max(spread)} of {b0 * bs}")


def test_twilight_equal_logits(K, dev):
    """Constant keys: every candidate has the same logit, so the top-p count
    is ceil(T / mass) and the lowest candidates win."""
    G, R, D, L, sink, recent, bs, b0 = 2, 4, 128, 2048, 16, 64, 16, 32
    keys = torch.full((G, L, D), 0.5, dtype=torch.float16)
    q = randn((G, R, D), "f32", seed=5)
    for mode, fixed in (("dynamic", 0), ("matched", 9)):
        _, _, sel, logits, desired, allocated, rows, counts = _layer(
            K, dev, "f16", G, R, D, L, sink, recent, bs, b0, 0.8, mode, fixed, 1.0, keys=keys, q=q)
        N = b0 * bs
        lg = logits.cpu().numpy()
        assert np.all(lg == lg[:, :, :1])
        # all masses equal: Z = N * 2^40, T = ceil(p24 * Z / 2^24)
        p24 = int(np.rint(np.float32(0.8) * np.float32(2 ** 24)))
        T = -(-(p24 * N * 2 ** 40) // 2 ** 24)
        want = -(-T // 2 ** 40)
        assert np.all(desired.cpu().numpy() == want)
        kb = to_bits(keys)
        P = oracle.selection_window(L, sink, recent)[2] // bs
        for g in range(G):
            pmin, pmax, packed, sc, mn = oracle.build_page_metadata(kb[g], "f16", sink, bs)
            ref = oracle.twilight_layer(q.numpy()[g], pmin[:P], pmax[:P], packed, sc, mn, "f16", length=L, sink=sink,
                                        recent=recent, block_size=bs, b0_pages=b0, top_p=0.8, budget_mode=mode,
                                        fixed_pages=fixed)
            assert np.array_equal(allocated[g].cpu().numpy(), ref["allocated"])
            n = int(counts[g])
            assert np.array_equal(rows[g, :n - 1].cpu().numpy(), ref["union"])


def test_twilight_logits_close_to_fp64(K, dev):
    """The INT4 estimate equals q . dequantized(k) / sqrt(D) to fp32 rounding."""
    G, R, D, L, sink, recent, bs, b0 = 2, 3, 128, 3000, 64, 256, 16, 48
    keys, q, sel, logits, *_ = _layer(K, dev, "bf16", G, R, D, L, sink, recent, bs, b0, 0.9, "dynamic", 0, 1.0)
    kb = to_bits(keys)
    for g in range(G):
        _, _, packed, sc, mn = oracle.build_page_metadata(kb[g], "bf16", sink, bs)
        deq = oracle.int4_dequantize(packed, sc, mn, "bf16").astype(np.float64)
        for r in range(R):
            pages = sel[g, r].cpu().numpy().astype(np.int64)
            pos = (sink + pages[:, None] * bs + np.arange(bs)).reshape(-1)
            want = deq[pos] @ q[g, r].double().numpy() / math.sqrt(D)
            got = logits[g, r].cpu().numpy().astype(np.float64)
            assert np.max(np.abs(got - want)) <= 1e-4 * (1.0 + np.max(np.abs(want)))


@pytest.mark.parametrize("bs,b0", [(16, 24), (8, 40)])
def test_twilight_union_pages_reaching_recent_window(K, dev, bs, b0):
    """Selections on pages that reach into the recent window (the page path of
    the union hands over to the token bitmap): the union counts a position
    the recent window also holds once, as np.unique over the oracle's
    top-p selections does."""
    G, R, L, sink, recent, top_p = 2, 4, 2048, 16, 64, 0.9
    _say(f"[twilight union overlap] bs={bs} b0={b0}")
    N = b0 * bs
    rng = np.random.default_rng(11 + bs)
    n_pages = (L - sink) // bs
    pages = np.empty((G, R, b0), np.int32)
    for g in range(G):
        for r in range(R):
            pages[g, r] = np.sort(rng.choice(n_pages, b0, replace=False))
        # head 0's last page: the last whole page, inside the recent window
        pages[g, 0] = np.append(np.sort(rng.choice(n_pages - 1, b0 - 1, replace=False)), n_pages - 1)
    logits = (rng.standard_normal((G, R, N)) * 3.0).astype(np.float32)
    rows = torch.full((G, L + 1), -5, dtype=torch.int32, device=dev)
    counts = torch.zeros((G,), dtype=torch.int32, device=dev)
    desired = torch.zeros((G, R), dtype=torch.int32, device=dev)
    K.twilight_select(torch.from_numpy(logits).to(dev), torch.from_numpy(pages).to(dev), top_p=top_p,
                      budget_mode="dynamic", rows=rows, row_counts=counts, desired=desired, sink=sink,
                      recent=recent, block_size=bs, length=L, append_position=L)
    torch.cuda.synchronize()
    sink_end, recent_start, _ = oracle.selection_window(L, sink, recent)
    offs = np.arange(bs)
    for g in range(G):
        assert pages[g, 0, -1] * bs + sink + bs > recent_start, "the case must reach the recent window"
        sel = []
        for r in range(R):
            d = oracle.top_p_count(logits[g, r], top_p)[0]
            assert int(desired[g, r]) == d, f"group {g} head {r}: desired"
            idx = oracle.topk_sorted(logits[g, r][None], d)[0]
            cand = (sink + pages[g, r][:, None] * bs + offs).reshape(-1)
            sel.append(cand[idx])
        union = np.unique(np.concatenate([np.arange(sink_end), *sel, np.arange(recent_start, L)]))
        n = int(counts[g])
        assert n == len(union) + 1, f"group {g}: union size {n - 1} vs {len(union)}"
        got = rows[g, :n].cpu().numpy()
        assert np.array_equal(got[:-1], union) and got[-1] == L


def test_twilight_candidates_past_the_limit_rejected(K, dev):
    """N = b0 * block_size above twilight_max_candidates() is refused before any
    launch (TW_EUNSUPPORTED), by every selection entry point."""
    cap = K.twilight_max_candidates()
    G, R, bs = 1, 2, 16
    b0 = cap // bs + 1
    logits = torch.zeros((G, R, b0 * bs), dtype=torch.float32, device=dev)
    sel = torch.arange(b0, dtype=torch.int32, device=dev).repeat(G, R, 1).contiguous()
    L = 64 + b0 * bs + 256
    rows = torch.zeros((G, L + 1), dtype=torch.int32, device=dev)
    counts = torch.zeros((G,), dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="twilight_select"):
        K.twilight_select(logits, sel, top_p=0.9, budget_mode="dynamic", rows=rows, row_counts=counts, sink=64,
                          recent=256, block_size=bs, length=L)
    slot_u = torch.zeros((G, R, b0), dtype=torch.int32, device=dev)
    prows = torch.zeros((G, R * b0), dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="twilight_select_pages"):
        K.twilight_select_pages(logits, sel, slot_u, prows, top_p=0.9, sink=64, recent=256, block_size=bs, length=L)
    torch.cuda.synchronize()
