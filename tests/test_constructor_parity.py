"""Constructor parity of TwilightMatchedBudgetOffloadedCache with the
reference (twilight_offload_cache.py:183-381): each ValueError condition the
reference raises before it builds the base cache raises the same message
here, and each combination the reference accepts passes validation.

The validation runs before the device is touched, so on a CPU-only machine an
accepted combination ends at the base cache's device check
("an operational ROCm device is required"), which is how these tests tell an
accepted combination from a rejected one.  On a device the accepted
combinations are constructed for real (tests/test_gpu_cache.py holds the
decode checks)."""

from __future__ import annotations

import pytest
import torch

BASE = dict(num_cache_entries=2, max_cache_len=64, head_dim=8, num_query_heads_per_kv=2, dtype=torch.bfloat16,
            device="cuda")

# The reference runner's zero-copy profile (twilight_offload_cache.py:264-270 requirements;
# scripts/run_ruler_partial_h2d_tpot_case_v1.py:101-106 passes
# --twilight-resident-snapshot-backend contiguous).
ZERO_COPY = dict(layer_batched_selection=True, gqa_groupwise_execution=True, gpu_compact_gqa_union=True,
                 cpu_flat_gather=True, direct_attention_layout=True, gather_h2d_chunks=4,
                 previous_token_resident_cache=True, resident_mapping_backend="gpu_bitmap",
                 resident_hit_copy_backend="triton", resident_snapshot_backend="contiguous",
                 resident_position_snapshot_backend="reference", resident_zero_copy=True)
CHUNKED = dict(layer_batched_selection=True, gqa_groupwise_execution=True, cpu_flat_gather=True,
               direct_attention_layout=True, gather_h2d_chunks=4)

REJECTED = [
    (dict(candidate_token_budget=0), "candidate_token_budget must be positive"),
    (dict(top_p=0.0), "top_p must be in"),
    (dict(top_p=1.5), "top_p must be in"),
    (dict(matched_budget_fraction=0.0), "matched_budget_fraction must be in"),
    (dict(budget_mode="fixed"), "budget_mode must be"),
    (dict(qk_backend="cuda"), "unknown Twilight QK backend"),
    (dict(qk_backend="triton"), "fused QK requires layer-batched selection"),
    (dict(exact_scan_graph=True, exact_top_p_graph=True), "select one exact Top-p graph scope"),
    (dict(resident_precompute_gpu_mapping=True), "precomputed GPU mapping requires mapped resident fast path"),
    (dict(vram_lazy_gpu_pack=True), "VRAM audit options require the mapped resident fast path"),
    (dict(vram_tight_resident_capacity=True), "VRAM audit options require the mapped resident fast path"),
    (dict(resident_zero_copy=True), "resident zero-copy requires resident cache"),
    (dict(resident_mapping_backend="cuda"), "unknown resident mapping backend"),
    (dict(resident_mapping_backend="native"), "native resident mapping requires resident cache"),
    (dict(resident_hit_copy_backend="cuda"), "unknown resident hit copy backend"),
    (dict(resident_hit_copy_backend="triton"), "Triton resident hit copy requires resident cache"),
    (dict(CHUNKED, previous_token_resident_cache=True, resident_mapping_backend="gpu_bitmap"),
     "compact hit indices require Triton hit copy"),
    (dict(resident_snapshot_backend="cuda"), "unknown resident snapshot backend"),
    (dict(resident_snapshot_backend="contiguous"), "alternate resident snapshot requires resident cache"),
    (dict(CHUNKED, previous_token_resident_cache=True, resident_snapshot_backend="contiguous"),
     "contiguous snapshot requires native_compact mapping and Triton hit copy"),
    (dict(resident_position_snapshot_backend="triton"), "unknown resident position snapshot backend"),
    (dict(resident_position_snapshot_backend="reference"),
     "reference position snapshot requires contiguous resident and GPU union"),
    (dict(ZERO_COPY, resident_mapping_backend="native_compact"),
     "resident zero-copy requires GPU bitmap mapping and contiguous GPU union"),
    (dict(resident_pack_hit_indices=True), "packed hit indices require contiguous resident"),
    (dict(new_kv_d2h_granularity="step"), "new KV D2H granularity must be"),
    (dict(gpu_compact_gqa_union=True), "GPU compact union requires GQA group execution"),
    (dict(gpu_union_validate_cpu=True), "GPU union CPU validation requires GPU compact union"),
    (dict(post_selection_groups_per_chunk=0), "post-selection groups per chunk must be positive"),
    (dict(CHUNKED, post_selection_pipeline=True), "post-selection pipeline requires"),
    (dict(cpu_run_gather=True), "run gather requires flat/direct/GQA chunk pipeline"),
    (dict(fused_quest_score=True), "fused Quest score requires layer-batched selection"),
    (dict(gather_h2d_chunks=-1), "gather_h2d_chunks must be nonnegative"),
    (dict(gather_h2d_chunks=2), "chunk pipeline requires flat gather, direct layout and GQA execution"),
    (dict(CHUNKED, cpu_native_gather=True), "chunk pipeline pilot uses PyTorch gather only"),
    (dict(early_gpu_metadata=True), "early GPU metadata requires GQA group execution"),
    (dict(direct_attention_layout=True), "native gather/direct layout requires flat gather"),
    (dict(cpu_native_gather=True), "native gather/direct layout requires flat gather"),
    (dict(cpu_flat_gather=True), "cpu_flat_gather requires GQA group execution"),
    (dict(layer_batched_selection=True, gqa_groupwise_execution=True, previous_token_resident_cache=True),
     "previous-token resident cache requires"),
    (dict(gqa_groupwise_execution=True), "GQA group-wise execution requires layer-batched selection"),
    (dict(layer_batched_selection=True, gqa_groupwise_execution=True, layer_flat_ragged_execution=True),
     "GQA group-wise and per-Query-head flat execution are exclusive"),
]

ACCEPTED = [
    dict(),
    dict(budget_mode="dynamic", candidate_token_budget=4096, top_p=0.95),
    dict(layer_batched_selection=True, qk_backend="triton"),
    dict(layer_batched_selection=True, qk_backend="triton_prepare", fused_quest_score=True),
    dict(exact_top_p_graph=True),
    dict(layer_batched_selection=True, gqa_groupwise_execution=True, gpu_compact_gqa_union=True,
         gpu_union_validate_cpu=True, early_gpu_metadata=True, batched_new_kv_d2h=True,
         new_kv_d2h_granularity="layer"),
    dict(CHUNKED),
    dict(CHUNKED, cpu_run_gather=True),
    dict(CHUNKED, gpu_compact_gqa_union=True, post_selection_pipeline=True, post_selection_groups_per_chunk=2),
    dict(CHUNKED, previous_token_resident_cache=True),
    dict(CHUNKED, previous_token_resident_cache=True, resident_mapping_backend="native_compact",
         resident_hit_copy_backend="triton", resident_snapshot_backend="contiguous",
         resident_pack_hit_indices=True),
    dict(ZERO_COPY),
    dict(ZERO_COPY, resident_precompute_gpu_mapping=True, vram_alias_history_staging=True, vram_lazy_gpu_pack=True,
         vram_ondemand_attention_capacity=True, vram_tight_resident_capacity=True),
    dict(layer_batched_selection=True, layer_flat_ragged_execution=True),
]


def _twilight():
    from headinfer.twilight_offload_cache import TwilightMatchedBudgetOffloadedCache

    return TwilightMatchedBudgetOffloadedCache


@pytest.mark.parametrize("kw,message", REJECTED, ids=[m[:40] for _, m in REJECTED])
def test_twilight_rejects_what_the_reference_rejects(kw, message):
    with pytest.raises(ValueError, match=message.replace("(", r"\(").replace(")", r"\)")):
        _twilight()(**BASE, **kw)


@pytest.mark.parametrize("kw", ACCEPTED, ids=[str(i) for i in range(len(ACCEPTED))])
def test_twilight_accepts_what_the_reference_accepts(kw):
    if torch.cuda.is_available():
        pytest.skip("constructed on the device by test_gpu_constructor_accepted")
    with pytest.raises(ValueError, match="an operational ROCm device is required"):
        _twilight()(**BASE, **kw)


def test_twilight_candidate_budget_limit():
    """Past tw_twilight_max_candidates() candidate tokens per head the
    selection cannot run, so the constructor refuses such a budget when the
    cache is long enough to reach it (and only then)."""
    from headinfer import kernels

    cap = kernels.twilight_max_candidates()
    assert cap == 16384
    long_cache = dict(BASE, max_cache_len=64 + cap + 2 * 16 + 256)
    for budget in (cap + 1, cap + 16, 4 * cap):
        with pytest.raises(ValueError, match="the Twilight selection takes at most 16384"):
            _twilight()(**long_cache, candidate_token_budget=budget)
    if torch.cuda.is_available():
        return
    # the widest selection fits: a budget of exactly the cap, or a cache too
    # short to give that many candidate pages
    for kw in (dict(long_cache, candidate_token_budget=cap), dict(BASE, candidate_token_budget=4 * cap)):
        with pytest.raises(ValueError, match="an operational ROCm device is required"):
            _twilight()(**kw)


def test_twilight_bad_windows_fail_in_the_quest_base():
    """Matched budgets with block_size 0 (or a negative sink, or no recent
    window) pass the Twilight checks and reach the Quest base, which refuses
    them with its ValueError (quest_offload_cache.py:47-53): the device check
    first, then the window check.  The candidate-budget limit must not divide
    by the block size ahead of it."""
    on_gpu = torch.cuda.is_available()
    want = "invalid sink/recent/block configuration" if on_gpu else "an operational ROCm device is required"
    dev = "cuda:0" if on_gpu else "cuda"
    for bad in (dict(block_size=0), dict(block_size=-16), dict(sink_tokens=-1), dict(recent_tokens=0)):
        with pytest.raises(ValueError, match=want):
            _twilight()(**dict(BASE, device=dev), budget_mode="matched", **bad)


def test_quest_accepts_more_than_eight_query_heads_per_kv():
    """The reference has no limit on query heads per KV head
    (quest_offload_cache.py:26-60); a 16-head group passes validation."""
    from headinfer.quest_offload_cache import QuestTopKOffloadedCache

    if torch.cuda.is_available():
        pytest.skip("a device is present")
    with pytest.raises(ValueError, match="an operational ROCm device is required"):
        QuestTopKOffloadedCache(**dict(BASE, num_query_heads_per_kv=16))


@pytest.mark.gpu
@pytest.mark.parametrize("kw", ACCEPTED, ids=[str(i) for i in range(len(ACCEPTED))])
def test_gpu_constructor_accepted(kw):
    cache = _twilight()(**dict(BASE, device="cuda:0"), **kw)
    snap = cache.state_snapshot()
    for name, value in kw.items():
        if f"requested_{name}" in snap:
            assert snap[f"requested_{name}"] == value
    assert cache.budget_fraction == cache.matched_budget_fraction
