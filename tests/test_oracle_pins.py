"""Pins of the CPU oracle (runs without a GPU).

The GPU kernels are checked against the oracle, so the oracle itself is
checked here against what fixes each function independently of its own code:
the golden vectors written from the reference's CPU helpers
(tests/golden/), closed forms, invariants, brute force on small inputs and
special cases chosen so that a plausible slip (a dropped term, a swapped
operand, a different summation order, an off-by-one window) fails.
"""

from __future__ import annotations

import json
import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
RNG = np.random.default_rng(1234)


def _bits_view(a: np.ndarray, dtype: str) -> np.ndarray:
    return a.view(np.float32) if dtype == "f32" else a.view(np.uint16)


# ------------------------------------------------------------------ INT4
@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_int4_pack_matches_reference_vectors(dtype):
    """affine_int4_pack / affine_int4_dequantize (twilight_offload_cache.py:
    25-47) on the reference's own outputs: codes, scale and minimum bits and
    the restored values, including a constant row, a tiny range, signed zeros
    and a row whose codes hit every rounding boundary."""
    z = np.load(GOLDEN / "int4_pack.npz")
    keys = _bits_view(z[f"{dtype}_keys"], dtype)
    T, D = keys.shape
    _, _, packed, scale, minimum = oracle.build_page_metadata(keys, dtype, sink=T, block_size=1, pages=False)
    assert np.array_equal(packed, z[f"{dtype}_packed"])
    want_scale = _bits_view(z[f"{dtype}_scale"], dtype)
    want_min = _bits_view(z[f"{dtype}_minimum"], dtype)
    assert np.array_equal(scale.view(np.uint8), want_scale.view(np.uint8))
    assert np.array_equal(minimum.view(np.uint8), want_min.view(np.uint8))
    restored = oracle.int4_dequantize(packed, scale, minimum, dtype)
    assert np.array_equal(restored.view(np.uint32), z[f"{dtype}_restored"].view(np.uint32))


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_int4_round_trip_bound(dtype):
    """|dequant - k| <= scale/2 + 1e-6 (scripts/test_twilight_offload_cache_v1.py:82-89)."""
    x = (RNG.standard_normal((64, 128)) * 3).astype(np.float32)
    keys = oracle.from_f32(x, dtype)
    kf = oracle.to_f32(keys, dtype)
    _, _, packed, scale, minimum = oracle.build_page_metadata(keys, dtype, sink=64, block_size=1, pages=False)
    deq = oracle.int4_dequantize(packed, scale, minimum, dtype)
    s = oracle.to_f32(scale, dtype)[:, None]
    assert np.all(np.abs(deq - kf) <= s / 2 + 1e-6 + 1e-6 * np.abs(kf))


# ---------------------------------------------------------- matched budgets
def test_matched_budget_counts_reference_vectors():
    """matched_budget_counts (twilight_offload_cache.py:50-86) and its tensor
    form (:89-130) on 47 cases produced by the reference functions."""
    cases = json.loads((GOLDEN / "matched_budget_counts.json").read_text())
    assert len(cases) >= 40
    for c in cases:
        got = oracle.matched_budget_counts(c["desired"], c["target"], c["capacities"])
        assert got == c["counts"], c
        if "counts_tensor" in c:
            assert got == c["counts_tensor"], c
        assert sum(got) == c["target"] and all(1 <= v <= cap for v, cap in zip(got, c["capacities"]))


def test_matched_budget_counts_rejects_infeasible():
    with pytest.raises(ValueError):
        oracle.matched_budget_counts([1, 2], 1, [4, 4])
    with pytest.raises(ValueError):
        oracle.matched_budget_counts([1, 2], 9, [4, 4])


# ------------------------------------------------------------ page min/max
def _total_order_minmax(x: np.ndarray, axis: int):
    """min/max in the IEEE total order (-0 < +0) via float64 with -0 shifted."""
    neg0 = (x == 0) & np.signbit(x)
    lo_key = np.where(neg0, -1e-300, x.astype(np.float64))
    idx_min = np.argmin(lo_key, axis=axis)
    idx_max = np.argmax(lo_key, axis=axis)
    return np.take_along_axis(x, np.expand_dims(idx_min, axis), axis).squeeze(axis), \
        np.take_along_axis(x, np.expand_dims(idx_max, axis), axis).squeeze(axis)


@pytest.mark.parametrize("dtype,T,D,sink,bs", [("f16", 203, 128, 64, 16), ("bf16", 90, 6, 5, 7),
                                               ("f32", 48, 32, 0, 16), ("bf16", 63, 8, 64, 16)])
def test_page_minmax_brute_force(dtype, T, D, sink, bs):
    """Complete pages [sink + p*bs, sink + (p+1)*bs) only (quest_offload_cache.py:276-289)."""
    x = RNG.standard_normal((T, D)).astype(np.float32)
    x[::7, 3 % D] = -0.0
    x[1::7, 3 % D] = 0.0
    keys = oracle.from_f32(x, dtype)
    kf = oracle.to_f32(keys, dtype)
    pmin, pmax, _, _, _ = oracle.build_page_metadata(keys, dtype, sink, bs, quant=False)
    P = max(0, (T - sink) // bs)
    assert pmin.shape[0] == P
    for p in range(P):
        lo, hi = _total_order_minmax(kf[sink + p * bs: sink + (p + 1) * bs], 0)
        assert np.array_equal(oracle.to_f32(pmin[p], dtype).view(np.uint32), lo.view(np.uint32))
        assert np.array_equal(oracle.to_f32(pmax[p], dtype).view(np.uint32), hi.view(np.uint32))


def test_page_minmax_nan_is_canonical():
    x = np.ones((32, 4), np.float32)
    x[5, 2] = np.nan
    keys = oracle.from_f32(x, "f16")
    pmin, pmax, _, _, _ = oracle.build_page_metadata(keys, "f16", 0, 16, quant=False)
    assert pmin[0, 2] == 0x7E00 and pmax[0, 2] == 0x7E00 and pmin[1, 2] == oracle.from_f32(np.float32(1), "f16")


# ------------------------------------------------------------- Quest score
def test_quest_score_is_an_upper_bound_and_close_to_float64():
    """score(p) >= q.k for every key of page p (the Quest bound) and equals
    sum_d where(q>0, max, min) * q to fp32 rounding."""
    G, R, T, D, bs = 2, 3, 16 * 40, 128, 16
    x = RNG.standard_normal((G, T, D)).astype(np.float32)
    keys = oracle.from_f32(x, "bf16")
    kf = oracle.to_f32(keys, "bf16")
    q = RNG.standard_normal((G, R, D)).astype(np.float32)
    pm = np.stack([oracle.build_page_metadata(keys[g], "bf16", 0, bs, quant=False)[0] for g in range(G)])
    px = np.stack([oracle.build_page_metadata(keys[g], "bf16", 0, bs, quant=False)[1] for g in range(G)])
    s = oracle.quest_score(q, pm, px, "bf16")
    lo, hi = oracle.to_f32(pm, "bf16").astype(np.float64), oracle.to_f32(px, "bf16").astype(np.float64)
    for g in range(G):
        for r in range(R):
            qq = q[g, r].astype(np.float64)
            exact = np.where(qq > 0, hi[g], lo[g]) @ qq
            mag = np.abs(np.where(qq > 0, hi[g], lo[g])) @ np.abs(qq)
            assert np.all(np.abs(s[g, r] - exact) <= 1e-6 * mag + 1e-30)
            dots = kf[g].astype(np.float64).reshape(-1, bs, D) @ qq
            assert np.all(dots.max(axis=1) <= s[g, r] + 1e-5 * mag)


def _score_one(terms: dict[int, float]) -> float:
    """Score of one page whose channel-d term is terms[d] (q = 1 on those channels)."""
    D = 128
    q = np.zeros((1, 1, D), np.float32)
    hi = np.zeros((1, 1, D), np.float32)
    for d, v in terms.items():
        q[0, 0, d] = 1.0
        hi[0, 0, d] = v
    return float(oracle.quest_score(q, hi.copy(), hi, "f32")[0, 0, 0])


def test_quest_score_summation_order():
    """The order of twilight_fused_quest.py:17-31: accumulator l sums channels
    l, l+32, l+64, l+96 in sequence, then an adjacent-pair tree over the 32
    accumulators.  2^24 + 1 rounds back to 2^24 in fp32, so each case below
    comes out differently under a different order."""
    big = float(2 ** 24)
    # same accumulator: (2^24 + 1) - 2^24 = 0 sequentially (a plain channel-order sum also gives 0) ...
    assert _score_one({0: big, 32: 1.0, 64: -big}) == 0.0
    # ... but channel 1 is another accumulator: 0 (acc 0) + 1 (acc 1) = 1, while a channel-order sum gives 0
    assert _score_one({0: big, 1: 1.0, 64: -big}) == 1.0
    # the tree pairs (0,1),(2,3): (1 + 0) + (2^24 - 2^24) = 1; a left-to-right sum over the accumulators gives 0
    assert _score_one({0: 1.0, 2: big, 3: -big}) == 1.0


@pytest.mark.parametrize("value", [0.0, 1.0, -1.0])
def test_quest_score_constant_pages_tie(value):
    """Equal pages score equally and top-k takes the lowest pages
    (scripts/test_twilight_fused_quest_v1.py:26-33 tie cases)."""
    q = RNG.standard_normal((1, 2, 128)).astype(np.float32)
    pages = np.full((1, 50, 128), value, np.float32)
    s = oracle.quest_score(q, pages, pages, "f32")
    assert np.all(s == s[:, :, :1])
    assert np.array_equal(oracle.topk_sorted(s, 7), np.tile(np.arange(7), (1, 2, 1)))


# ------------------------------------------------------------------ top-k
def _brute_topk(row: np.ndarray, k: int) -> list[int]:
    def key(i):
        v = float(row[i])
        return (0 if math.isnan(v) else 1, 0.0 if math.isnan(v) else -v, i)
    return sorted(sorted(range(len(row)), key=key)[:k])


@pytest.mark.parametrize("P,k", [(1, 1), (9, 3), (50, 50), (300, 17), (2028, 128)])
def test_topk_brute_force(P, k):
    row = RNG.integers(-5, 6, P).astype(np.float32)  # many ties
    if P > 5:
        row[2] = np.nan
        row[4] = -0.0
        row[5] = 0.0
    got = oracle.topk_sorted(row[None], k)[0]
    assert list(got) == _brute_topk(row, k)


# --------------------------------------------------------------- row plan
@pytest.mark.parametrize("L,sink,recent,bs,R,k", [(4096, 64, 256, 16, 4, 16), (300, 4, 9, 7, 3, 5),
                                                  (40, 64, 256, 16, 2, 1), (1000, 0, 1, 8, 8, 30)])
def test_row_plan_is_the_set_union(L, sink, recent, bs, R, k):
    """sink ++ union of the heads' pages expanded ++ recent ++ decode row,
    ascending, with the heads that see each row (quest_offload_cache.py:
    403-511, union as in scripts/test_twilight_offload_cache_v1.py:291-294)."""
    sink_end, recent_start, eligible = oracle.selection_window(L, sink, recent)
    P = eligible // bs
    if P == 0:
        sel = np.zeros((R, 0), np.int64)
        k = 0
    else:
        k = min(k, P)
        sel = np.stack([np.sort(RNG.choice(P, k, replace=False)) for _ in range(R)])
    rows, masks = oracle.quest_row_plan(sel, P, sink, recent, bs, L, append_position=L)
    per_head = [set(range(sink_end)) | set(range(recent_start, L))
                | {sink + p * bs + i for p in sel[r] for i in range(bs)} for r in range(R)]
    union = sorted(set().union(*per_head))
    assert list(rows[:-1]) == union and rows[-1] == L
    for t, m in zip(rows[:-1], masks[:-1]):
        assert m == sum(1 << r for r in range(R) if t in per_head[r])


def test_selection_window_and_budget_closed_form():
    """quest_offload_cache.py:326-346 at the 4K and 32K layers."""
    assert oracle.selection_window(4096, 64, 256) == (64, 3841, 3777)
    assert oracle.quest_budget(4096, 64, 256, 16, 0.05, (4096 - 64) // 16) == (236, 12)
    assert oracle.quest_budget(32768, 64, 256, 16, 0.0625, (32768 - 64) // 16) == (2028, 127)
    assert oracle.selection_window(100, 64, 256) == (64, 64, 0)
    assert oracle.selection_window(10, 64, 256) == (10, 10, 0)


# --------------------------------------------------------------- Twilight
def test_det_exp_against_libm():
    xs = np.concatenate([np.linspace(-28, 0, 20001, dtype=np.float32), np.float32([-1e-30, -0.0, 0.0])])
    for x in xs:
        e = oracle.det_exp(float(x))
        want = math.exp(float(x))
        # rounding t = x*log2(e) to fp32 costs half an ulp of t, i.e. up to
        # 2^(floor(log2|t|) - 24) * ln 2 relative; fp32 log2(e) is 1.34e-8 low
        # (|x| * 1.34e-8 relative); the degree-6 polynomial ~1e-7
        t = abs(float(x)) * 1.4426950408889634
        t_err = 2.0 ** (math.floor(math.log2(t)) - 24) * math.log(2) if t >= 2 ** -20 else 0.0
        assert abs(e - want) <= (t_err + 1.4e-8 * abs(float(x)) + 3e-7) * want, (x, e, want)
    assert oracle.det_exp(0.0) == 1.0
    assert oracle.det_exp(-28.01) == 0.0 and oracle.det_exp(float("-inf")) == 0.0
    assert oracle.det_exp(float("nan")) == 0.0


def _brute_top_p(logits: np.ndarray, top_p: float) -> int:
    lmax = float(np.max(logits))
    masses = [oracle.mass(float(v), lmax) for v in logits]
    z = sum(masses)
    p24 = int(np.rint(np.float32(top_p) * np.float32(2 ** 24)))
    need = -(-(p24 * z) // 2 ** 24)
    order = sorted(range(len(logits)), key=lambda i: (-float(logits[i]), i))
    cum = 0
    for c, i in enumerate(order):
        cum += masses[i]
        if cum >= need:
            return c + 1
    return len(logits)


@pytest.mark.parametrize("N,top_p,spread", [(1, 0.95, 1.0), (16, 0.5, 0.1), (400, 0.95, 3.0), (4096, 0.99, 5.0),
                                            (333, 1.0, 2.0), (64, 0.3, 0.0)])
def test_top_p_count_brute_force_and_float64(N, top_p, spread):
    """ExactTopPGraph (twilight_exact_top_p_graph.py:19-32): the smallest
    count whose largest softmax probabilities reach top_p."""
    logits = (RNG.standard_normal(N) * spread).astype(np.float32)
    if N > 8:
        logits[3] = logits[5]  # a tie
    d, z = oracle.top_p_count(logits, top_p)
    assert d == _brute_top_p(logits, top_p)
    lmax = float(np.max(logits))
    assert z == sum(oracle.mass(float(v), lmax) for v in logits)
    # float64 softmax + cumsum: the same count up to the 2^-40 mass quantum at the boundary
    p = np.exp(logits.astype(np.float64) - logits.max())
    p /= p.sum()
    cum = np.cumsum(np.sort(p)[::-1])
    d64 = int(np.searchsorted(cum, float(np.float32(top_p)) - 1e-12, side="left")) + 1
    assert abs(d - min(d64, N)) <= 1


def test_top_p_count_closed_forms():
    one_hot = np.full(100, -60.0, np.float32)
    one_hot[37] = 5.0
    assert oracle.top_p_count(one_hot, 0.95)[0] == 1
    for N, p in ((10, 0.5), (7, 0.3), (128, 0.95), (1000, 0.999)):
        uniform = np.zeros(N, np.float32)
        assert oracle.top_p_count(uniform, p)[0] == math.ceil(Fraction(int(np.rint(np.float32(p) * 2 ** 24)), 2 ** 24) * N)
    assert oracle.top_p_threshold(10 * 2 ** 40, 0.5) == 5 * 2 ** 40
    assert oracle.top_p_threshold(3, 1.0) == 3


def _fp32_top_p(logits: torch.Tensor, top_p: float) -> tuple[torch.Tensor, torch.Tensor]:
    """The reference's fp32 op sequence, restated with torch on the CPU
    (twilight_offload_cache.py:1275-1309, twilight_exact_top_p_graph.py:19-32):
    descending argsort, softmax of the sorted logits, one 1-D cumsum per head,
    searchsorted(right=False) + 1 against top_p, clamped to the row."""
    order = torch.argsort(logits, dim=-1, descending=True)
    probs = torch.softmax(torch.gather(logits, -1, order), dim=-1)
    cum = torch.stack([row.cumsum(dim=0) for row in probs.flatten(0, -2)]).view_as(probs)
    thr = torch.full((*cum.shape[:-1], 1), top_p, dtype=cum.dtype)
    desired = torch.searchsorted(cum.contiguous(), thr, right=False).squeeze(-1) + 1
    return desired.clamp_max(logits.shape[-1]), order


@pytest.mark.parametrize("N,spread,top_p", [(4096, 1.5, 0.95), (4096, 4.0, 0.95), (1024, 0.5, 0.9),
                                            (4096, 2.5, 0.99), (256, 8.0, 0.95)])
def test_top_p_count_against_reference_fp32_rule(N, spread, top_p):
    """The exact integer-mass count against the reference's fp32 count on the
    same logits.  They agree wherever fp32 rounding cannot decide; where they
    differ, every cumulative probability between the two counts (float64) lies
    within the fp32 rounding budget of top_p (N ulps at 1.0), and the kept
    tokens are the same whenever the counts are."""
    rows = 64
    g = torch.Generator().manual_seed(N + int(10 * spread))
    logits = torch.randn(rows, N, generator=g) * spread
    logits[:, :N // 8] += 2.0 * spread * torch.rand(rows, N // 8, generator=g)  # a peaked head of the row
    ref, order = _fp32_top_p(logits, top_p)
    tol = N * 2.0 ** -24
    agree = 0
    for r in range(rows):
        lg = logits[r].numpy()
        d, _ = oracle.top_p_count(lg, top_p)
        dr = int(ref[r])
        if d == dr:
            agree += 1
            ours = sorted(range(N), key=lambda i: (-float(lg[i]), i))[:d]
            assert set(ours) == set(order[r, :d].tolist())
            continue
        p64 = np.exp(lg.astype(np.float64) - float(lg.max()))
        cum = np.cumsum(np.sort(p64)[::-1] / p64.sum())
        for k in range(min(d, dr), max(d, dr)):
            assert abs(cum[k - 1] - float(np.float32(top_p))) <= tol, (r, d, dr, k)
    assert agree >= rows * 9 // 10, agree


def _int4_qk_crafted(values: dict[int, int], q_of: dict[int, float], scale: float = 1.0,
                     minimum: float = 0.0, D: int = 64) -> float:
    """One candidate with codes `values` (others 0), fp32 scale/minimum, against q."""
    codes = np.zeros(D, np.int64)
    for d, v in values.items():
        codes[d] = int(v)
    packed = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)[None]
    q = np.zeros(D, np.float32)
    for d, v in q_of.items():
        q[d] = v
    return float(oracle.int4_qk(q, packed, np.float32([scale]), np.float32([minimum]), "f32",
                                np.zeros(1, np.int64), 1.0)[0])


def test_qfix_closed_forms():
    """q~ = Q * 2^(E - 22), E the frexp exponent of max |q|, Q rounded half to even."""
    Q, qs, shift, ok = oracle.qfix(np.float32([1.0, -0.5, 0.0, 2.0 ** -30]))
    assert ok and shift == 1 - 22 and Q.tolist() == [2 ** 21, -(2 ** 20), 0, 0] and qs == 2 ** 21 - 2 ** 20
    Q, _, shift, _ = oracle.qfix(np.float32([3.0, 2.5 * 2.0 ** -20, 3.5 * 2.0 ** -20]))   # E = 2: x 2^20
    assert shift == -20 and Q.tolist() == [3 * 2 ** 20, 2, 4]                             # 2.5 -> 2, 3.5 -> 4
    Q, qs, shift, ok = oracle.qfix(np.zeros(8, np.float32))
    assert ok and qs == 0 and shift == 0 and not Q.any()
    assert not oracle.qfix(np.float32([1.0, np.nan]))[3] and not oracle.qfix(np.float32([np.inf, 0.0]))[3]


def test_int4_qk_defined_arithmetic():
    """logit = qk_scale * ((scale * ldexp(S, shift)) + (min * ldexp(sum Q, shift))),
    S = sum code * Q exact.  Each case separates the definition from a
    plausible variant."""
    # S = 15 * 128 * 2^21 > 2^31: an int32 accumulator would wrap
    assert _int4_qk_crafted({d: 15 for d in range(128)}, {d: 1.0 for d in range(128)}, D=128) == 1920.0
    # Q rounds half to even: q_1 * 2^21 = 2.5 -> 2 (half away from zero gives 3)
    assert _int4_qk_crafted({1: 1}, {0: 1.0, 1: 2.5 * 2.0 ** -21}) == 2 * 2.0 ** -21
    # the exponent is frexp's (max |q| = 1 -> E = 1, q x 2^21): q_1 = 1.25 * 2^-22 -> Q_1 = 1,
    # i.e. 2^-21 (scaling by 2^22 would give 2^-22)
    assert _int4_qk_crafted({1: 1}, {0: 1.0, 1: 1.25 * 2.0 ** -22}) == 2.0 ** -21
    # two rounded products then a rounded sum (a fused multiply-add gives 2^-22 + 2^-43)
    got = _int4_qk_crafted({0: 1, 1: 1}, {0: 1.0, 1: 2.0 ** -21}, scale=1.0 + 2.0 ** -22, minimum=-1.0)
    assert got == 2.0 ** -22
    # a non-finite query gives NaN, an all-zero query the minimum times zero
    assert math.isnan(_int4_qk_crafted({0: 3}, {0: float("inf")}))
    assert _int4_qk_crafted({0: 3}, {}, scale=2.0, minimum=5.0) == 0.0


@pytest.mark.parametrize("dtype,D", [("bf16", 128), ("f16", 64), ("f32", 256), ("bf16", 4)])
def test_int4_qk_close_to_float64_and_one_hot_exact(dtype, D):
    x = (RNG.standard_normal((300, D)) * 2).astype(np.float32)
    keys = oracle.from_f32(x, dtype)
    _, _, packed, scale, minimum = oracle.build_page_metadata(keys, dtype, 300, 1, pages=False)
    deq = oracle.int4_dequantize(packed, scale, minimum, dtype).astype(np.float64)
    rows = RNG.choice(300, 100, replace=False).astype(np.int64)
    qs = np.float32(1.0 / math.sqrt(D))
    q = RNG.standard_normal(D).astype(np.float32)
    got = oracle.int4_qk(q, packed, scale, minimum, dtype, rows, float(qs))
    want = deq[rows] @ q.astype(np.float64) * float(qs)
    mag = np.abs(deq[rows]) @ np.abs(q.astype(np.float64)) * float(qs)
    # q~ differs from q by at most 2^(E-23) <= 2^-22 max|q| per channel
    qerr = np.abs(deq[rows]).sum(axis=1) * float(np.abs(q).max()) * 2.0 ** -22 * float(qs)
    assert np.all(np.abs(got - want) <= qerr + 4e-7 * mag + 1e-30)
    for d in (0, D // 2 + 1, D - 1):
        e = np.zeros(D, np.float32)
        e[d] = 1.0
        got = oracle.int4_qk(e, packed, scale, minimum, dtype, rows, float(qs))
        assert np.array_equal(got, (deq[rows, d].astype(np.float32) * qs).astype(np.float32))


def test_twilight_layer_invariants():
    """Per-head selections have the allocated sizes, matched budgets sum to
    the target, and the union is sink | selections | recent."""
    T, D, sink, recent, bs, R = 1500, 64, 16, 32, 8, 3
    keys = oracle.from_f32(RNG.standard_normal((T, D)).astype(np.float32), "bf16")
    pmin, pmax, packed, sc, mn = oracle.build_page_metadata(keys, "bf16", sink, bs)
    _, recent_start, eligible = oracle.selection_window(T, sink, recent)
    P = eligible // bs
    q = (RNG.standard_normal((R, D)) * 3).astype(np.float32)
    for mode, fixed in (("dynamic", 0), ("matched", 12)):
        out = oracle.twilight_layer(q, pmin[:P], pmax[:P], packed, sc, mn, "bf16", length=T, sink=sink,
                                    recent=recent, block_size=bs, b0_pages=40, top_p=0.9, budget_mode=mode,
                                    fixed_pages=fixed)
        N = 40 * bs
        assert out["logits"].shape == (R, N)
        for r in range(R):
            assert len(out["selected"][r]) == out["allocated"][r]
            assert set(out["selected"][r]) <= set(out["candidates"][r])
            assert out["desired"][r] == oracle.top_p_count(out["logits"][r], 0.9)[0]
        if mode == "matched":
            assert int(out["allocated"].sum()) == fixed * bs * R
        else:
            assert np.array_equal(out["allocated"], out["desired"])
        want = set(range(sink)) | set(range(recent_start, T)) | set().union(*map(set, out["selected"]))
        assert list(out["union"]) == sorted(want)


# --------------------------------------------------------------- attention
def test_decode_attention_oracle_matches_torch_sdpa():
    """decode_attention (float64) == torch SDPA math in fp32 (the reference's
    decode_reference_attention.py:55-68), with and without head masks."""
    R, N, D = 4, 777, 128
    q = RNG.standard_normal((R, D)).astype(np.float32)
    k = RNG.standard_normal((N, D)).astype(np.float32)
    v = RNG.standard_normal((N, D)).astype(np.float32)
    scale = 1.0 / math.sqrt(D)
    got = oracle.decode_attention(q, k, v, scale)
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q)[:, None, None], torch.from_numpy(k)[None, None].expand(R, 1, N, D),
        torch.from_numpy(v)[None, None].expand(R, 1, N, D), scale=scale)[:, 0, 0].double().numpy()
    assert np.max(np.abs(got - ref)) < 1e-5
    masks = RNG.integers(0, 16, N).astype(np.uint8)
    masks[0] = 15
    got = oracle.decode_attention(q, k, v, scale, masks)
    for r in range(R):
        vis = ((masks >> r) & 1).astype(bool)
        ref = oracle.decode_attention(q[r:r + 1], k[vis], v[vis], scale)[0]
        assert np.max(np.abs(got[r] - ref)) < 1e-12
