"""The fallback branches of the fused Twilight kernels against the oracle.

The fused selection (twilight_select_fused: twilight_topp_head_kernel, and
with matched budgets twilight_matched_rec_kernel) takes one-pass histogram
fast paths that give up, block-uniformly, when

* the B0 top-k's score keys span no finite positive range, or more than 64
  keys fall in the boundary bin (then block_topk, the digit search);
* the top-p's logit keys span no finite positive range, the logits carry no
  mass (NaN), or more than 64 keys fall in the boundary mass bin (then
  block_top_mass, the general search);
* the matched allocation's top-k hits the same conditions on the logits
  (then block_topk).

Random N(0,1) keys never reach these branches.  Each case below builds
inputs that do -- equal Quest scores, clustered scores with one far page,
equal logits, clustered logits with far rows, NaN and infinite queries --
asserts on the CPU that the fast path's condition fails for them, and holds
B0 pages, logits (bit patterns), top-p counts, allocations and the union
record to oracle.twilight_layer (twilight_offload_cache.py:1144-1354 in this
build's defined orders), for dynamic and matched budgets; the union-record
attention is held to 2e-3 abs + 1e-2 rel of float64 over the oracle's rows
for every head with a finite query."""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
import torch

import oracle
from helpers import to_bits

pytestmark = pytest.mark.gpu

BS, SINK, RECENT, D = 16, 64, 256, 128
FAST_BINS = 512   # bins of the one-pass fast paths
WAVE = 64         # boundary keys a fast path ranks in one wavefront


def _say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def K():
    from headinfer import kernels

    return kernels


def _boundary_bin_count(values: np.ndarray, weights: np.ndarray, need: float) -> int | None:
    """Keys in the bin where the weight of the bins above it first reaches
    `need` (bins linear in the value over [min, max], FAST_BINS of them, fp32
    like the kernels), or None when the range is not finite and positive --
    the fast paths give up on either a count above 64 or a None."""
    v = np.asarray(values, np.float32)
    if np.isnan(v).any():
        return None
    vmin, vmax = np.float32(v.min()), np.float32(v.max())
    rng = np.float32(vmax - vmin)
    if not (np.isfinite(vmin) and np.isfinite(vmax) and np.isfinite(rng) and rng > 0):
        return None
    scale = np.float32(FAST_BINS) / rng
    if not np.isfinite(scale):
        return None
    b = np.minimum(((v - vmin) * scale).astype(np.int64), FAST_BINS - 1)
    cnt = np.bincount(b, minlength=FAST_BINS)
    w = np.bincount(b, weights=np.asarray(weights, np.float64), minlength=FAST_BINS)
    acc = 0.0
    for bi in range(FAST_BINS - 1, -1, -1):
        if acc + w[bi] >= need:
            return int(cnt[bi])
        acc += w[bi]
    return int(cnt[0])


def topk_fast_gives_up(values: np.ndarray, k: int) -> bool:
    if k >= values.size:
        return False
    c = _boundary_bin_count(values, np.ones(values.size), k)
    return c is None or c > WAVE


def top_p_fast_gives_up(logits: np.ndarray, top_p: float) -> bool:
    lmax = np.float32(np.max(np.where(np.isnan(logits), -np.inf, logits)))
    mass = np.array([oracle.mass(float(x), float(lmax)) if not np.isnan(x) else 0 for x in logits], np.float64)
    z = int(sum(int(m) for m in mass))
    need = oracle.top_p_threshold(z, top_p)
    if need == 0:
        return True
    c = _boundary_bin_count(logits, mass, float(need))
    return c is None or c > WAVE


def _decode_record(rec, P):
    rec = rec.astype(np.int64) & 0xFFFFFFFF
    nb = 2 * ((P + 63) // 64)
    off = (nb + 3) & ~3
    bits = np.array([(rec[p >> 5] >> (p & 31)) & 1 for p in range(32 * nb)], bool)
    masks = np.array([(rec[off + (p >> 1)] >> (16 * (p & 1))) & 0xFFFF for p in range(P)], np.int64)
    return bits, masks


def _record_of(kept_pos, P):
    masks = np.zeros(P, np.int64)
    for p in kept_pos:
        page, i = divmod(int(p) - SINK, BS)
        assert 0 <= page < P
        masks[page] |= 1 << i
    return masks


class Case:
    """Crafted inputs of G groups at one length L: keys/values [G, L+8, D]
    bf16, page metadata and INT4 keys (built from the keys, then optionally
    overridden), queries [G, R, D] fp32 (bf16 values)."""

    def __init__(self, K, dev, G, R, L, seed):
        self.G, self.R, self.L = G, R, L
        self.P = oracle.selection_window(L, SINK, RECENT)[2] // BS
        gen = torch.Generator(device=dev).manual_seed(seed)
        Lmax = L + 8
        bf = torch.bfloat16
        self.k = (torch.randn((G, Lmax, D), generator=gen, device=dev) * 1.5).to(bf)
        self.v = torch.randn((G, Lmax, D), generator=gen, device=dev).to(bf)
        self.q = (torch.randn((G, R, D), generator=gen, device=dev) * 2).to(bf).float()
        self.cur_k = torch.randn((G, D), generator=gen, device=dev).to(bf)
        self.cur_v = torch.randn((G, D), generator=gen, device=dev).to(bf)
        Pm = (L - SINK) // BS
        self.pmin = torch.zeros((G, Pm, D), dtype=bf, device=dev)
        self.pmax = torch.zeros_like(self.pmin)
        self.packed = torch.zeros((G, Lmax, D // 2), dtype=torch.uint8, device=dev)
        self.scale = torch.zeros((G, Lmax), dtype=bf, device=dev)
        self.minimum = torch.zeros_like(self.scale)
        K.build_page_metadata(self.k[:, :L], sink=SINK, block_size=BS, page_min=self.pmin, page_max=self.pmax,
                              packed=self.packed[:, :L], scale=self.scale[:, :L], minimum=self.minimum[:, :L])
        self.gen = gen


def run_fused(K, dev, c: Case, b0, top_p, mode, fixed=0, attend=True, tag=""):
    """The fused selection over the case, every output against the oracle;
    returns the oracle's per-group results."""
    G, R, L, P = c.G, c.R, c.L, c.P
    matched = mode == "matched"
    words = K.union_record_words(P)
    rec = torch.full((G, (words + 3) & ~3), -1, dtype=torch.int32, device=dev)   # garbage: the score launch clears it
    sel = torch.zeros((G, R, b0), dtype=torch.int32, device=dev)
    logits = torch.zeros((G, R, b0 * BS), dtype=torch.float32, device=dev)
    desired = torch.zeros((G, R), dtype=torch.int32, device=dev)
    allocated = torch.full((G, R), -7, dtype=torch.int32, device=dev) if matched else None
    _say(f"[fallback] {tag}: G={G} R={R} L={L} b0={b0} top_p={top_p} {mode} fixed={fixed}")
    K.twilight_select_fused(c.q, c.pmin[:, :P], c.pmax[:, :P], c.packed, c.scale, c.minimum, b0, rec, top_p=top_p,
                            sink=SINK, recent=RECENT, block_size=BS, length=L, desired=desired, sel_pages=sel,
                            logits=logits, budget_mode=mode, target_total=fixed * BS * R if matched else 0,
                            allocated=allocated)
    k_att, v_att = c.k.clone(), c.v.clone()
    out = None
    if attend:
        out = K.decode_attention_union(c.q.to(torch.bfloat16), k_att, v_att, rec, P, max_pages=min(P, R * b0),
                                       sink=SINK, recent=RECENT, block_size=BS, length=L, append=True,
                                       cur_k=c.cur_k, cur_v=c.cur_v)
    torch.cuda.synchronize()
    rec_h, sel_h, log_h, des_h = rec.cpu().numpy(), sel.cpu().numpy(), logits.cpu().numpy(), desired.cpu().numpy()
    refs = []
    for gi in range(G):
        ref = oracle.twilight_layer(c.q[gi].cpu().numpy(), to_bits(c.pmin[gi, :P]), to_bits(c.pmax[gi, :P]),
                                    c.packed[gi].cpu().numpy(), to_bits(c.scale[gi]), to_bits(c.minimum[gi]), "bf16",
                                    length=L, sink=SINK, recent=RECENT, block_size=BS, b0_pages=b0, top_p=top_p,
                                    budget_mode=mode, fixed_pages=fixed)
        assert np.array_equal(sel_h[gi], ref["pages"]), (tag, gi, "B0 pages")
        assert np.array_equal(log_h[gi].view(np.uint32), ref["logits"].astype(np.float32).view(np.uint32)), \
            (tag, gi, "logits")
        assert np.array_equal(des_h[gi], ref["desired"]), (tag, gi, des_h[gi], ref["desired"])
        if matched:
            assert np.array_equal(allocated[gi].cpu().numpy(), ref["allocated"]), (tag, gi, ref["allocated"])
        bits, masks = _decode_record(rec_h[gi], P)
        want = _record_of(np.unique(np.concatenate(ref["selected"])), P)
        assert np.array_equal(masks, want), (tag, gi, "record row masks")
        assert np.array_equal(bits[:P], want != 0) and not bits[P:].any(), (tag, gi, "record page bits")
        refs.append(ref)
    if attend:
        got = out.float().cpu().numpy()
        for gi in range(G):
            kept = refs[gi]["union"].astype(np.int64)
            keys = torch.cat([c.k[gi, kept].float(), c.cur_k[gi:gi + 1].float()]).cpu().numpy()
            vals = torch.cat([c.v[gi, kept].float(), c.cur_v[gi:gi + 1].float()]).cpu().numpy()
            ref_o = oracle.decode_attention(c.q[gi].cpu().numpy(), keys, vals, 1.0 / math.sqrt(D))
            for r in range(R):
                if not np.isfinite(c.q[gi, r].cpu().numpy()).all():
                    continue   # a non-finite query attends to NaN in both
                err = np.abs(got[gi, r] - ref_o[r])
                assert np.all(err <= 2e-3 + 1e-2 * np.abs(ref_o[r])), (tag, gi, r, float(err.max()))
        # the decode token's row went into the slab at L
        assert torch.equal(k_att[:, L].view(torch.int16), c.cur_k.view(torch.int16))
    _say(f"[fallback] {tag} ok: desired {des_h.tolist()}")
    return refs


def _scores(c: Case, gi: int) -> np.ndarray:
    return oracle.quest_score(c.q[gi][None].cpu().numpy(), to_bits(c.pmin[gi, :c.P])[None],
                              to_bits(c.pmax[gi, :c.P])[None], "bf16")[0]


MODES = [("dynamic", 0), ("matched", 12)]


@pytest.mark.parametrize("mode,fixed", MODES)
def test_b0_topk_fallback_equal_scores(K, dev, mode, fixed):
    """Every page has the same min/max, so every Quest score is equal: the
    head kernel's B0 top-k takes block_topk and keeps the lowest page ids.
    The INT4 keys are the random keys' (the top-p fast path runs)."""
    c = Case(K, dev, 2, 4, 6000, seed=101)
    c.pmin.fill_(-0.5)
    c.pmax.fill_(0.75)
    b0 = 64
    for gi in range(c.G):
        s = _scores(c, gi)
        assert all(topk_fast_gives_up(s[r], b0) for r in range(c.R))
    refs = run_fused(K, dev, c, b0, 0.95, mode, fixed, tag=f"equal scores {mode}")
    assert all(np.array_equal(r["pages"], np.tile(np.arange(b0), (c.R, 1))) for r in refs)


@pytest.mark.parametrize("mode,fixed", MODES)
def test_b0_topk_fallback_clustered_scores(K, dev, mode, fixed):
    """Every page's extrema are one shared pattern plus a few ulps of jitter,
    so every score is near sum |q_d| (|b_d| + 1) (about 370), while one page
    with min = max = 0 scores 0: the boundary bin of the one-pass histogram
    holds every other page (> 64), so the head kernel's B0 top-k takes
    block_topk."""
    c = Case(K, dev, 2, 4, 6000, seed=102)
    G, P = c.G, c.P
    gen = torch.Generator(device=dev).manual_seed(7)
    base = torch.randn((G, 1, D), generator=gen, device=dev)
    jitter = torch.randint(0, 4, (G, c.pmin.shape[1], D), generator=gen, device=dev).float() * 2.0 ** -7
    c.pmax.copy_((base.abs() + 1.0 + jitter).to(torch.bfloat16))
    c.pmin.copy_((-base.abs() - 1.0 - jitter).to(torch.bfloat16))
    c.pmax[:, 5] = 0.0
    c.pmin[:, 5] = 0.0
    b0 = 64
    for gi in range(G):
        s = _scores(c, gi)
        assert all(topk_fast_gives_up(s[r], b0) for r in range(c.R)), gi
        assert all(np.unique(s[r]).size > b0 for r in range(c.R))   # not merely all equal
    run_fused(K, dev, c, b0, 0.95, mode, fixed, tag=f"clustered scores {mode}")


@pytest.mark.parametrize("mode,fixed", MODES)
def test_top_p_fallback_equal_logits(K, dev, mode, fixed):
    """Every INT4 row has code 0 and the same scale and minimum, so every
    logit of a head is the same: the top-p takes the general search (and
    matched budgets the allocation's block_topk), keeping the lowest
    candidates.  The page metadata is the random keys' (B0 fast path)."""
    c = Case(K, dev, 2, 4, 6000, seed=103)
    c.packed.zero_()
    c.scale.fill_(0.125)
    c.minimum.fill_(0.5)
    b0 = 64
    refs = run_fused(K, dev, c, b0, 0.9, mode, fixed, tag=f"equal logits {mode}")
    for ref in refs:
        for r in range(c.R):
            assert np.unique(ref["logits"][r]).size == 1
            assert top_p_fast_gives_up(ref["logits"][r], 0.9)
            if mode == "matched":
                assert topk_fast_gives_up(ref["logits"][r], int(ref["allocated"][r]))
            # equal masses: the smallest count whose mass reaches 0.9 Z
            assert abs(int(ref["desired"][r]) - 0.9 * b0 * BS) <= 1


@pytest.mark.parametrize("mode,fixed", MODES)
def test_top_p_fallback_clustered_logits(K, dev, mode, fixed):
    """Random codes at a tiny scale put every logit of a head within a hair
    of the others, while every 64th row carries a minimum of -32 (the query
    is positive, so those logits sit far below): the boundary mass bin holds
    thousands of distinct logits, so the top-p takes the general search and
    the matched allocation's top-k takes block_topk."""
    c = Case(K, dev, 2, 4, 9000, seed=104)
    gen = torch.Generator(device=dev).manual_seed(9)
    c.q = (torch.randn(c.q.shape, generator=gen, device=dev).abs() + 0.05).to(torch.bfloat16).float()
    c.packed.copy_(torch.randint(0, 256, c.packed.shape, generator=gen, device=dev).to(torch.uint8))
    c.scale.fill_(2.0 ** -10)
    c.minimum.zero_()
    c.minimum[:, ::64] = -32.0
    b0 = 128
    refs = run_fused(K, dev, c, b0, 0.95, mode, fixed, tag=f"clustered logits {mode}")
    for ref in refs:
        for r in range(c.R):
            lg = ref["logits"][r]
            assert np.unique(lg).size > 1000
            assert top_p_fast_gives_up(lg, 0.95)
            if mode == "matched":
                assert topk_fast_gives_up(lg, int(ref["allocated"][r]))


@pytest.mark.parametrize("mode,fixed", MODES)
def test_fallbacks_non_finite_queries(K, dev, mode, fixed):
    """A head with a NaN in its query scores every page NaN (B0: block_topk,
    the lowest pages) and estimates every logit NaN (no mass: top-p keeps
    one candidate); a head with +inf scores pages +-inf or NaN and gets NaN
    logits too.  The group's other heads run the fast paths beside them."""
    c = Case(K, dev, 2, 4, 6000, seed=105)
    c.q[0, 1, 5] = float("nan")
    c.q[1, 2, 0] = float("inf")
    b0 = 64
    for gi, r in ((0, 1), (1, 2)):
        assert not np.isfinite(_scores(c, gi)[r]).all()   # no finite key range: block_topk
    refs = run_fused(K, dev, c, b0, 0.95, mode, fixed, tag=f"non-finite queries {mode}")
    for gi, r in ((0, 1), (1, 2)):
        assert np.isnan(refs[gi]["logits"][r]).all()
        assert top_p_fast_gives_up(refs[gi]["logits"][r], 0.95)
        assert refs[gi]["desired"][r] == 1
    assert np.array_equal(refs[0]["pages"][1], np.arange(b0))   # all NaN: the lowest pages


def test_fused_matched_refuses_target_past_b0(K, dev):
    """With device lengths the matched target grows with the length while B0
    stays at b0 pages; where the longest group's target would pass them the
    reference's allocation raises (twilight_offload_cache.py:58-59), and so
    does the wrapper, instead of clamping on the device."""
    c = Case(K, dev, 1, 4, 6000, seed=106)
    P = c.P
    words = K.union_record_words(P)
    rec = torch.zeros((1, (words + 3) & ~3), dtype=torch.int32, device=dev)
    lens = torch.tensor([c.L], dtype=torch.int32, device=dev)
    # fixed = ceil(0.05 * 5681 / 16) = 18 pages a head: 8 B0 pages are too few
    with pytest.raises(ValueError, match="infeasible"):
        K.twilight_select_fused(c.q, c.pmin[:, :P], c.pmax[:, :P], c.packed, c.scale, c.minimum, 8, rec,
                                top_p=0.95, sink=SINK, recent=RECENT, block_size=BS, length=c.L, lengths=lens,
                                budget_mode="matched", matched_fraction=0.05)
    K.twilight_select_fused(c.q, c.pmin[:, :P], c.pmax[:, :P], c.packed, c.scale, c.minimum, 18, rec,
                            top_p=0.95, sink=SINK, recent=RECENT, block_size=BS, length=c.L, lengths=lens,
                            budget_mode="matched", matched_fraction=0.05)
    torch.cuda.synchronize()
