"""Twilight selection (Quest B0 -> INT4 QK -> top-p -> budgets -> GQA union)
on one MI355X, with the reference's call surface.

Reference: twilight_offload_cache.py -- the pure helpers affine_int4_pack /
affine_int4_dequantize / matched_budget_counts(_tensor) (:25-130) and
TwilightMatchedBudgetOffloadedCache (:133-3743): constructor keywords and
defaults (candidate_token_budget 8192, top_p 0.95, matched_budget_fraction
0.05, budget_mode "matched"), prepare_layer_selection,
update_layer_gqa_group_ragged, the traces and state_snapshot.

decode_layer selects a decoder layer in two launches on the device with
dynamic budgets -- tw_twilight_select_fused: the Quest score and the INT4
estimate of every scored row for the group's heads, then one block per head
for the B0 pages, the exact top-p and the group's union record -- and three
with matched budgets (the allocation and each head's top-allocated rows in
one more launch); more than 8 query heads per KV head run as sub-groups of at
most 8 whose records are ORed (with matched budgets every sub-group's
allocation launch reads the counts of all the group's heads).  The attention
then reads the record's rows from the slab (HBM or zero-copy host) with the
decode token's append fused.  Under a selection or budget trace (which
records the row list), for shapes outside the fused kernels (D != 128, pages
other than 16 rows, more than 8192 candidate pages or B0 tokens), or with
matched budgets over more than 64 query heads per KV head, the general path
runs instead: tw_quest_select (B0 pages + union
plan), tw_twilight_qk, tw_twilight_select (counts, budgets, per-head
selection, the token union as a row list), then the row attention; both
attend the same rows.  The update APIs (update_layer_gqa_group_ragged and the
per-entry update) take the general path and gather the selected rows into
the varlen attention layout.  The reference's many execution variants
(qk_backend, CPU union / gather flavours, graphs, pipelines, resident caches)
choose between implementations of the same selection; they are accepted and
validated like the reference does, recorded in state_snapshot, and run these
paths.
"""

from __future__ import annotations

import hashlib
import math
from typing import Any, Dict, Optional, Sequence

import torch

from . import kernels
from .quest_offload_cache import QuestTopKOffloadedCache, _window

__all__ = [
    "affine_int4_pack",
    "affine_int4_dequantize",
    "matched_budget_counts",
    "matched_budget_counts_tensor",
    "TwilightMatchedBudgetOffloadedCache",
]


# ----------------------------------------------------------------- helpers
def affine_int4_pack(keys: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per-token asymmetric INT4 of [tokens, even head_dim] keys on the GPU:
    (packed uint8 [T, D/2] low nibble = even channel, scale [T], minimum [T])
    bit-exact with twilight_offload_cache.py:25-37."""
    return kernels.affine_int4_pack(keys)


def affine_int4_dequantize(packed: torch.Tensor, scale: torch.Tensor, minimum: torch.Tensor) -> torch.Tensor:
    """f32(code) * f32(scale) + f32(minimum) (twilight_offload_cache.py:40-47)."""
    return kernels.affine_int4_dequantize(packed, scale, minimum)


def matched_budget_counts(desired: list[int], target_total: int, capacities: list[int]) -> list[int]:
    """Largest-remainder rescaling of per-head top-p counts to an exact total
    (twilight_offload_cache.py:50-86).

    Every head keeps at least one; the remaining target is split in
    proportion to desired in float64, floors first (capped by capacity), then
    single increments go to the largest fractional remainder (ties: larger
    desired, then lower index), an increment zeroing that head's remainder;
    an excess is taken from the smallest (desired, index) above one."""
    n = len(desired)
    if not desired or n != len(capacities):
        raise ValueError("desired and capacities must be non-empty and aligned")
    if min(desired) <= 0 or min(capacities) <= 0:
        raise ValueError("desired counts and capacities must be positive")
    if target_total < n or target_total > sum(capacities):
        raise ValueError("target_total is infeasible")
    spare = target_total - n
    weight = float(sum(float(d) for d in desired))
    share = [spare * float(d) / weight for d in desired]
    counts = [1 + min(capacities[i] - 1, int(math.floor(share[i]))) for i in range(n)]
    total = sum(counts)
    while total < target_total:
        open_heads = [i for i in range(n) if counts[i] < capacities[i]]
        if not open_heads:
            raise AssertionError("unable to fill matched budget")
        pick = open_heads[0]
        for i in open_heads[1:]:
            fi, fp = share[i] - math.floor(share[i]), share[pick] - math.floor(share[pick])
            if fi > fp or (fi == fp and desired[i] > desired[pick]):
                pick = i
        counts[pick] += 1
        share[pick] = math.floor(share[pick])
        total += 1
    while total > target_total:
        over = [i for i in range(n) if counts[i] > 1]
        if not over:
            raise AssertionError("unable to reduce matched budget")
        pick = over[0]
        for i in over[1:]:
            if desired[i] < desired[pick]:
                pick = i
        counts[pick] -= 1
        total -= 1
    return counts


def matched_budget_counts_tensor(desired: torch.Tensor, target_total: int, capacity: int) -> torch.Tensor:
    """matched_budget_counts for every row of desired [groups, heads] at once,
    for the unsaturated case target_total <= capacity (no capacity clamp can
    act), without a host sync (twilight_offload_cache.py:89-130).

    Head i of a row gets 1 + floor(share_i) plus one more if fewer than
    `deficit` heads precede it in the order (remainder desc, desired desc,
    index asc); the precedence is counted pairwise over the heads."""
    if desired.ndim != 2 or desired.shape[1] <= 0:
        raise ValueError("desired must be [groups, query_heads]")
    heads = int(desired.shape[1])
    if target_total < heads or target_total > capacity:
        raise ValueError("target_total must be between head count and capacity")
    d = desired.to(torch.float64)
    share = (target_total - heads) * d / d.sum(dim=-1, keepdim=True)
    base = torch.floor(share)
    counts = 1 + base.to(torch.long)
    deficit = target_total - counts.sum(dim=-1, keepdim=True)
    frac = share - base
    fi, fj = frac.unsqueeze(-1), frac.unsqueeze(-2)       # [G, i, j]
    di, dj = desired.unsqueeze(-1), desired.unsqueeze(-2)
    idx = torch.arange(heads, device=desired.device)
    j_before_i = (fj > fi) | ((fj == fi) & ((dj > di) | ((dj == di) & (idx.view(1, 1, -1) < idx.view(1, -1, 1)))))
    rank = j_before_i.sum(dim=-1)
    return counts + (rank < deficit).to(counts.dtype)


# ------------------------------------------------------------------- cache
class TwilightMatchedBudgetOffloadedCache(QuestTopKOffloadedCache):
    """Quest B0 + INT4 QK + top-p with matched or dynamic budgets."""

    def __init__(
        self,
        *,
        candidate_token_budget: int = 8192,
        top_p: float = 0.95,
        matched_budget_fraction: float = 0.05,
        budget_mode: str = "matched",
        gqa_groupwise_execution: bool = False,
        detailed_selection_profile: bool = False,
        qk_backend: str = "pytorch",
        exact_scan_graph: bool = False,
        exact_top_p_graph: bool = False,
        cpu_flat_gather: bool = False,
        cpu_bitmap_union: bool = False,
        cpu_native_gather: bool = False,
        direct_attention_layout: bool = False,
        early_gpu_metadata: bool = False,
        gather_h2d_chunks: int = 0,
        reuse_quant_metadata: bool = False,
        fused_final_indices: bool = False,
        fused_quest_score: bool = False,
        skip_unused_host_views: bool = False,
        cpu_run_gather: bool = False,
        previous_token_resident_cache: bool = False,
        resident_mapping_backend: str = "torch",
        resident_hit_copy_backend: str = "torch",
        resident_snapshot_backend: str = "torch",
        resident_position_snapshot_backend: str = "clone",
        resident_pack_hit_indices: bool = False,
        resident_zero_copy: bool = False,
        resident_precompute_gpu_mapping: bool = False,
        vram_alias_history_staging: bool = False,
        vram_lazy_gpu_pack: bool = False,
        vram_ondemand_attention_capacity: bool = False,
        vram_tight_resident_capacity: bool = False,
        gpu_compact_gqa_union: bool = False,
        gpu_union_validate_cpu: bool = False,
        batched_new_kv_d2h: bool = False,
        new_kv_d2h_granularity: str = "token",
        post_selection_pipeline: bool = False,
        post_selection_groups_per_chunk: int = 1,
        **kwargs: Any,
    ) -> None:
        # Validation follows twilight_offload_cache.py:183-381 condition by
        # condition, in the same order and with the same messages, so a
        # configuration fails here exactly when it fails in the reference.
        if candidate_token_budget <= 0:
            raise ValueError("candidate_token_budget must be positive")
        if not 0.0 < top_p <= 1.0:
            raise ValueError("top_p must be in (0, 1]")
        if not 0.0 < matched_budget_fraction <= 1.0:
            raise ValueError("matched_budget_fraction must be in (0, 1]")
        if budget_mode not in {"matched", "dynamic"}:
            raise ValueError("budget_mode must be 'matched' or 'dynamic'")
        num_query_heads_per_kv = int(kwargs["num_query_heads_per_kv"])
        layer_batched_selection = bool(kwargs.get("layer_batched_selection", False))
        if qk_backend not in {"pytorch", "triton", "triton_prepare"}:
            raise ValueError("unknown Twilight QK backend")
        if qk_backend != "pytorch" and not layer_batched_selection:
            raise ValueError("fused QK requires layer-batched selection")
        if exact_scan_graph and exact_top_p_graph:
            raise ValueError("select one exact Top-p graph scope")
        if resident_precompute_gpu_mapping and not resident_zero_copy:
            raise ValueError("precomputed GPU mapping requires mapped resident fast path")
        if any((vram_alias_history_staging, vram_lazy_gpu_pack, vram_ondemand_attention_capacity,
                vram_tight_resident_capacity)) and not resident_zero_copy:
            raise ValueError("VRAM audit options require the mapped resident fast path")
        if resident_zero_copy and not previous_token_resident_cache:
            raise ValueError("resident zero-copy requires resident cache")
        if resident_mapping_backend not in {"torch", "native", "native_compact", "gpu_bitmap"}:
            raise ValueError("unknown resident mapping backend")
        if resident_mapping_backend != "torch" and not previous_token_resident_cache:
            raise ValueError("native resident mapping requires resident cache")
        if resident_hit_copy_backend not in {"torch", "triton"}:
            raise ValueError("unknown resident hit copy backend")
        if resident_hit_copy_backend != "torch" and not previous_token_resident_cache:
            raise ValueError("Triton resident hit copy requires resident cache")
        if resident_mapping_backend in {"native_compact", "gpu_bitmap"} and resident_hit_copy_backend != "triton":
            raise ValueError("compact hit indices require Triton hit copy")
        if resident_snapshot_backend not in {"torch", "triton", "contiguous"}:
            raise ValueError("unknown resident snapshot backend")
        if resident_snapshot_backend != "torch" and not previous_token_resident_cache:
            raise ValueError("alternate resident snapshot requires resident cache")
        if resident_snapshot_backend == "contiguous" and (
                resident_mapping_backend not in {"native_compact", "gpu_bitmap"}
                or resident_hit_copy_backend != "triton"):
            raise ValueError("contiguous snapshot requires native_compact mapping and Triton hit copy")
        if resident_position_snapshot_backend not in {"clone", "reference"}:
            raise ValueError("unknown resident position snapshot backend")
        if resident_position_snapshot_backend == "reference" and (
                resident_snapshot_backend != "contiguous" or not gpu_compact_gqa_union):
            raise ValueError("reference position snapshot requires contiguous resident and GPU union")
        if resident_zero_copy and not (resident_mapping_backend == "gpu_bitmap"
                                       and resident_snapshot_backend == "contiguous"
                                       and resident_position_snapshot_backend == "reference"
                                       and gpu_compact_gqa_union):
            raise ValueError("resident zero-copy requires GPU bitmap mapping and contiguous GPU union")
        if resident_pack_hit_indices and (resident_snapshot_backend != "contiguous"
                                          or resident_mapping_backend != "native_compact"):
            raise ValueError("packed hit indices require contiguous resident and native_compact mapping")
        if new_kv_d2h_granularity not in {"layer", "token"}:
            raise ValueError("new KV D2H granularity must be 'layer' or 'token'")
        if gpu_compact_gqa_union and not gqa_groupwise_execution:
            raise ValueError("GPU compact union requires GQA group execution")
        if gpu_union_validate_cpu and not gpu_compact_gqa_union:
            raise ValueError("GPU union CPU validation requires GPU compact union")
        if int(post_selection_groups_per_chunk) <= 0:
            raise ValueError("post-selection groups per chunk must be positive")
        if post_selection_pipeline and not (gpu_compact_gqa_union and gqa_groupwise_execution and cpu_flat_gather
                                            and direct_attention_layout and gather_h2d_chunks > 0
                                            and not cpu_native_gather and not cpu_run_gather
                                            and not previous_token_resident_cache):
            raise ValueError("post-selection pipeline requires the current GPU-union GQA flat/direct/chunk path "
                             "without native/run gather or resident reuse")
        if cpu_run_gather and (not (cpu_flat_gather and direct_attention_layout and gqa_groupwise_execution
                                    and gather_h2d_chunks > 0) or cpu_native_gather):
            raise ValueError("run gather requires flat/direct/GQA chunk pipeline without native gather")
        if fused_quest_score and not layer_batched_selection:
            raise ValueError("fused Quest score requires layer-batched selection")
        if int(gather_h2d_chunks) < 0:
            raise ValueError("gather_h2d_chunks must be nonnegative")
        if gather_h2d_chunks and not (cpu_flat_gather and direct_attention_layout and gqa_groupwise_execution):
            raise ValueError("chunk pipeline requires flat gather, direct layout and GQA execution")
        if gather_h2d_chunks and cpu_native_gather:
            raise ValueError("chunk pipeline pilot uses PyTorch gather only")
        if early_gpu_metadata and not gqa_groupwise_execution:
            raise ValueError("early GPU metadata requires GQA group execution")
        if (cpu_native_gather or direct_attention_layout) and not (cpu_flat_gather and gqa_groupwise_execution):
            raise ValueError("native gather/direct layout requires flat gather and GQA group execution")
        if cpu_flat_gather and not gqa_groupwise_execution:
            raise ValueError("cpu_flat_gather requires GQA group execution")
        if previous_token_resident_cache and not (gqa_groupwise_execution and cpu_flat_gather
                                                  and direct_attention_layout and gather_h2d_chunks > 0
                                                  and not cpu_native_gather and not cpu_run_gather):
            raise ValueError("previous-token resident cache requires the current GQA flat/direct/chunk path "
                             "without native/run gather")
        layer_flat_ragged_execution = bool(kwargs.get("layer_flat_ragged_execution", False))
        if gqa_groupwise_execution and not layer_batched_selection:
            raise ValueError("GQA group-wise execution requires layer-batched selection")
        if gqa_groupwise_execution and layer_flat_ragged_execution:
            raise ValueError("GQA group-wise and per-Query-head flat execution are exclusive")
        # The Quest base selects with the matched fraction, and sizes its
        # per-head packs for the largest Twilight selection
        # (twilight_offload_cache.py:353-370).
        kwargs["budget_fraction"] = matched_budget_fraction
        if budget_mode == "dynamic":
            max_cache_len = int(kwargs["max_cache_len"])
            sink_tokens = int(kwargs.get("sink_tokens", 64))
            block_size = int(kwargs.get("block_size", 16))
            max_pages = math.ceil(max(0, max_cache_len - sink_tokens) / block_size)
            required_pages = min(max_pages, math.ceil(candidate_token_budget / block_size))
            kwargs["max_selected_history_fraction"] = required_pages / max_pages if max_pages else 1.0
        else:
            kwargs["max_selected_history_fraction"] = min(1.0, matched_budget_fraction * num_query_heads_per_kv)
        # The one limit the reference does not have: a top-p block holds at
        # most kernels.twilight_max_candidates() candidate tokens per head
        # (B0 pages x page size).  A budget the longest cache would take past
        # it is refused here rather than at the first decode step.  Windows the
        # Quest base refuses (quest_offload_cache.py:52) reach it unchecked, so
        # they fail with its error, as in the reference.
        block_size = int(kwargs.get("block_size", 16))
        sink_tokens = int(kwargs.get("sink_tokens", 64))
        recent_tokens = int(kwargs.get("recent_tokens", 256))
        widest = 0
        if block_size > 0 and sink_tokens >= 0 and recent_tokens > 0:
            _, _, eligible = _window(int(kwargs["max_cache_len"]), sink_tokens, recent_tokens)
            widest = min(eligible // block_size, max(1, math.ceil(candidate_token_budget / block_size))) * block_size
        if widest > kernels.twilight_max_candidates():
            raise ValueError(
                f"candidate_token_budget {candidate_token_budget} gives {widest} candidate tokens per head at "
                f"max_cache_len {kwargs['max_cache_len']}; the Twilight selection takes at most "
                f"{kernels.twilight_max_candidates()}")
        super().__init__(**kwargs)
        if cpu_bitmap_union and not gqa_groupwise_execution:
            raise ValueError("cpu_bitmap_union requires GQA group execution")
        # The reference's host natives behind the CPU variants; the union,
        # gather and attention of this cache run on the device, so these are
        # held for callers that use them directly.
        if cpu_run_gather:
            from .cpu_kv_run_gather import CpuKVRunGather
            self._cpu_run_gather = CpuKVRunGather()
        if cpu_native_gather:
            from .cpu_kv_gather import CpuKVGather
            self._cpu_kv_gather = CpuKVGather()
        if cpu_bitmap_union:
            from .cpu_token_union import CpuTokenUnion
            self._cpu_token_union = CpuTokenUnion(self.geometry.max_cache_len)
        self.candidate_token_budget = int(candidate_token_budget)
        self.top_p = float(top_p)
        # The previous-token resident cache (twilight_offload_cache.py:2457-2608,
        # 3323-3470): with a host slab, the fused decode keeps each group's last
        # union rows in HBM, row by row, with the sink and recent windows, and
        # reads only the other rows over the host link.  An HBM slab needs no
        # such cache, and the fused shapes bound it (16-bit K/V, head_dim 128,
        # 16-row pages, at most 8 query heads per KV head); elsewhere the flag
        # is validated and recorded only.
        self.previous_token_resident_cache = bool(previous_token_resident_cache)
        self._resident_active = (self.previous_token_resident_cache and self.kv_residency == "host"
                                 and self.block_size == 16 and self.geometry.head_dim == 128
                                 and self.dtype in (torch.float16, torch.bfloat16)
                                 and self.num_query_heads_per_kv <= 8)
        # ... and on the reference's own GQA-group path (update_layer_gqa_group_ragged),
        # where it lives in the reference: each layer's previous packed union
        # stays in HBM and rows it holds are copied from there
        self._gqa_resident: dict[int, dict] = {}
        self.matched_budget_fraction = float(matched_budget_fraction)
        self.budget_mode = budget_mode
        self.gqa_groupwise_execution = bool(gqa_groupwise_execution)
        self.detailed_selection_profile = bool(detailed_selection_profile)
        self.qk_backend = qk_backend
        self.exact_scan_graph = bool(exact_scan_graph)
        self.exact_top_p_graph = bool(exact_top_p_graph)
        self.cpu_flat_gather = bool(cpu_flat_gather)
        self.cpu_bitmap_union = bool(cpu_bitmap_union)
        self.cpu_native_gather = bool(cpu_native_gather)
        self.direct_attention_layout = bool(direct_attention_layout)
        self.early_gpu_metadata = bool(early_gpu_metadata)
        self.gather_h2d_chunks = int(gather_h2d_chunks)
        self.reuse_quant_metadata = bool(reuse_quant_metadata)
        self.fused_final_indices = bool(fused_final_indices)
        self.fused_quest_score = bool(fused_quest_score)
        self.skip_unused_host_views = bool(skip_unused_host_views)
        self.cpu_run_gather = bool(cpu_run_gather)
        self.resident_zero_copy = bool(resident_zero_copy)
        self.resident_precompute_gpu_mapping = bool(resident_precompute_gpu_mapping)
        self.resident_mapping_backend = resident_mapping_backend
        self.resident_hit_copy_backend = resident_hit_copy_backend
        self.resident_snapshot_backend = resident_snapshot_backend
        self.resident_position_snapshot_backend = resident_position_snapshot_backend
        self.resident_pack_hit_indices = bool(resident_pack_hit_indices)
        self.gpu_union_validate_cpu = bool(gpu_union_validate_cpu)
        self.batched_new_kv_d2h = bool(batched_new_kv_d2h)
        self.new_kv_d2h_granularity = new_kv_d2h_granularity
        self.post_selection_pipeline = bool(post_selection_pipeline)
        self.post_selection_groups_per_chunk = int(post_selection_groups_per_chunk)
        self._variant_flags = dict(
            qk_backend=qk_backend, resident_mapping_backend=resident_mapping_backend,
            resident_hit_copy_backend=resident_hit_copy_backend, resident_snapshot_backend=resident_snapshot_backend,
            resident_position_snapshot_backend=resident_position_snapshot_backend,
            new_kv_d2h_granularity=new_kv_d2h_granularity, exact_scan_graph=exact_scan_graph,
            exact_top_p_graph=exact_top_p_graph,
            cpu_flat_gather=cpu_flat_gather, cpu_bitmap_union=cpu_bitmap_union, cpu_native_gather=cpu_native_gather,
            direct_attention_layout=direct_attention_layout, early_gpu_metadata=early_gpu_metadata,
            gather_h2d_chunks=gather_h2d_chunks, reuse_quant_metadata=reuse_quant_metadata,
            fused_final_indices=fused_final_indices, fused_quest_score=fused_quest_score,
            skip_unused_host_views=skip_unused_host_views, cpu_run_gather=cpu_run_gather,
            previous_token_resident_cache=previous_token_resident_cache,
            resident_pack_hit_indices=resident_pack_hit_indices, resident_zero_copy=resident_zero_copy,
            resident_precompute_gpu_mapping=resident_precompute_gpu_mapping,
            vram_alias_history_staging=vram_alias_history_staging, vram_lazy_gpu_pack=vram_lazy_gpu_pack,
            vram_ondemand_attention_capacity=vram_ondemand_attention_capacity,
            vram_tight_resident_capacity=vram_tight_resident_capacity, gpu_compact_gqa_union=gpu_compact_gqa_union,
            gpu_union_validate_cpu=gpu_union_validate_cpu, batched_new_kv_d2h=batched_new_kv_d2h,
            post_selection_pipeline=post_selection_pipeline,
            post_selection_groups_per_chunk=post_selection_groups_per_chunk)
        self.gpu_compact_gqa_union = bool(gpu_compact_gqa_union)
        self._packed: Optional[torch.Tensor] = None   # [E, T_prompt, D/2] uint8
        self._qscale: Optional[torch.Tensor] = None   # [E, T_prompt]
        self._qmin: Optional[torch.Tensor] = None
        # per entry: the prepared layer state and the group index within it
        self._prepared_layer: Dict[int, tuple[dict, int]] = {}
        self._group_union_trace: list[dict[str, Any]] = []
        self._budget_trace: list[dict[str, Any]] = []
        self._capture_budget_trace = False
        # decode_layer with dynamic budgets runs the fused selection (union
        # record) when the shapes allow; False keeps the union-row path
        self.fused_decode = True
        self._fused_bufs: Optional[tuple[torch.Tensor, torch.Tensor]] = None
        self._flat_union_keys: Optional[torch.Tensor] = None
        self._flat_union_values: Optional[torch.Tensor] = None
        self._dma = None  # HostGatherPipeline of post_selection_pipeline (host slabs)

    # ------------------------------------------------------------ metadata
    def _build_metadata(self, entry: int, key_states: torch.Tensor) -> None:
        """Page min/max and per-token INT4 keys of the prompt in one launch
        (twilight_offload_cache.py:925-936)."""
        keys = key_states[0, 0].contiguous()
        T = int(keys.shape[0])
        E, D = self.geometry.num_entries, self.geometry.head_dim
        pages = (T - self.sink_tokens) // self.block_size if T > self.sink_tokens else 0
        if self._page_min is None:
            rows = max(T, self.geometry.max_cache_len) if self.update_metadata_on_decode else T
            self._page_min = torch.empty((E, self._metadata_page_capacity(pages), D), dtype=self.dtype,
                                         device=self.device)
            self._page_max = torch.empty_like(self._page_min)
            self._packed = torch.empty((E, rows, D // 2), dtype=torch.uint8, device=self.device)
            self._qscale = torch.empty((E, rows), dtype=self.dtype, device=self.device)
            self._qmin = torch.empty_like(self._qscale)
        assert self._packed is not None and self._qscale is not None and self._qmin is not None
        kernels.build_page_metadata(keys, sink=self.sink_tokens, block_size=self.block_size,
                                    page_min=self._page_min[entry] if pages else None,
                                    page_max=self._page_max[entry] if pages else None,
                                    packed=self._packed[entry], scale=self._qscale[entry],
                                    minimum=self._qmin[entry])

    def _update_decode_metadata(self, entries: Sequence[int], position: int) -> None:
        """The decode row's INT4 code and the page it completes, if any."""
        if not self.update_metadata_on_decode or self._page_min is None:
            return
        start = self._phase_start()
        for e0, n in self._runs(entries):
            kernels.update_page_metadata(self._key_cache, first_entry=e0, n_entries=n, position=position,
                                         sink=self.sink_tokens, block_size=self.block_size,
                                         page_min=self._page_min, page_max=self._page_max, packed=self._packed,
                                         scale=self._qscale, minimum=self._qmin)
        self._phase_end("metadata_update", start)

    # --------------------------------------------------------------- budgets
    def resident_pages(self) -> "kernels.ResidentPages":
        """The HBM resident cache of every entry (allocated on first use):
        slots for the widest union the B0 budget allows (R x B0 pages), a map
        over every page the metadata can hold, and the sink and recent
        windows."""
        if self._resident is None:
            if self._page_min is None:
                raise RuntimeError("prompt metadata is missing")
            pages = max(1, int(self._page_min.shape[1]))
            b0 = max(1, math.ceil(self.candidate_token_budget / self.block_size))
            slots = max(1, min(pages, self.num_query_heads_per_kv * b0, 0xffff))
            self._resident = kernels.ResidentPages(self.geometry.num_entries, slots, pages, self.geometry.head_dim,
                                                   self.dtype, self.device, sink=self.sink_tokens,
                                                   recent=self.recent_tokens)
        return self._resident

    def _twilight_budgets(self, old_length: int) -> tuple[int, int, int, int, int]:
        """(sink_end, recent_start, candidate_pages, fixed_pages, b0_pages) of
        twilight_offload_cache.py:1019-1083."""
        sink_end, recent_start, eligible = _window(old_length, self.sink_tokens, self.recent_tokens)
        cand = eligible // self.block_size
        fixed = min(cand, max(1, math.ceil(self.matched_budget_fraction * eligible / self.block_size)))
        b0 = min(cand, max(1, math.ceil(self.candidate_token_budget / self.block_size)))
        if self._page_min is None or self._packed is None:
            raise RuntimeError("Twilight prompt metadata is missing")
        cand = min(cand, int(self._page_min.shape[1]))
        return sink_end, recent_start, cand, min(fixed, cand), min(b0, cand)

    # -------------------------------------------------------------- selection
    def _select_layer(self, entries: Sequence[int], q: torch.Tensor, old_length: int) -> dict:
        """Both Twilight stages for the entries of one layer, on the device.
        Returns the layer state: union rows [G, L+1] / row_counts [G] (without
        the decode token), desired / allocated [G, R], per-head candidate
        bitmaps and the B0 pages."""
        G, R = len(entries), self.num_query_heads_per_kv
        sink_end, recent_start, cand, fixed, b0 = self._twilight_budgets(old_length)
        rows = torch.empty((G, old_length + 1), dtype=torch.int32, device=self.device)
        counts = torch.empty((G,), dtype=torch.int32, device=self.device)
        state: dict[str, Any] = {"entries": tuple(entries), "old_length": old_length, "rows": rows,
                                 "counts": counts, "b0": b0, "fixed": fixed, "max_count": old_length}
        if cand == 0 or fixed == 0 or b0 == 0:
            prot = torch.cat([torch.arange(sink_end), torch.arange(recent_start, old_length)]).to(torch.int32)
            rows[:, :prot.numel()].copy_(prot.to(self.device).expand(G, -1))
            counts.fill_(int(prot.numel()))
            state.update(desired=None, allocated=None, head_bits=None, pages=None)
            return state
        pmin, pmax = self._metadata(entries, cand)
        if R > 8:
            state.update(self._select_heads_split(entries, q, old_length, pmin, pmax, b0, fixed))
            return state
        N = b0 * self.block_size
        sel = torch.empty((G, R, b0), dtype=torch.int32, device=self.device)
        width = min(cand, R * b0)
        plan_pages = torch.empty((G, width), dtype=torch.int32, device=self.device)
        plan_masks = torch.empty((G, width), dtype=torch.uint8, device=self.device)
        plan_counts = torch.empty((G,), dtype=torch.int32, device=self.device)
        start = self._phase_start()
        kernels.quest_select(q, pmin, pmax, b0, sel_pages=sel, plan_pages=plan_pages, plan_masks=plan_masks,
                             plan_counts=plan_counts)
        self._phase_end("twilight_quest_b0", start)
        packed, qscale, qmin = self._quant(entries)
        start = self._phase_start()
        logits = kernels.twilight_qk(q, packed, qscale, qmin, plan_pages, plan_masks, plan_counts, b0,
                                     sink=self.sink_tokens, block_size=self.block_size)
        self._phase_end("twilight_int4_qk", start)
        desired = torch.empty((G, R), dtype=torch.int32, device=self.device)
        allocated = torch.empty((G, R), dtype=torch.int32, device=self.device)
        head_bits = torch.empty((G, R, (N + 31) // 32), dtype=torch.int32, device=self.device)
        start = self._phase_start()
        kernels.twilight_select(logits, sel, top_p=self.top_p, budget_mode=self.budget_mode,
                                target_total=fixed * self.block_size * R, rows=rows, row_counts=counts,
                                desired=desired, allocated=allocated, head_bits=head_bits, sink=self.sink_tokens,
                                recent=self.recent_tokens, block_size=self.block_size, length=old_length)
        self._phase_end("twilight_top_p_union", start)
        state.update(desired=desired, allocated=allocated, head_bits=head_bits, pages=sel, logits=logits)
        return state

    def _select_heads_split(self, entries: Sequence[int], q: torch.Tensor, old_length: int, pmin: torch.Tensor,
                            pmax: torch.Tensor, b0: int, fixed: int) -> dict:
        """Both stages for more than 8 query heads per KV head: the kernels
        take at most 8 heads per group, so the heads run in sub-groups of at
        most 8.  Each head's B0 pages, logits and top-p count depend on that
        head alone, so they are the same as in one call.  Matched budgets are
        shared by all R heads of a group (twilight_offload_cache.py:50-86):
        the desired counts of every sub-group are gathered, allocated over the
        R heads with matched_budget_counts, and each sub-group then keeps its
        heads' given allocations.  The group's union is the sorted union of
        the sub-groups' unions (each holds the sink and recent windows)."""
        G, R = q.shape[0], q.shape[1]
        bs, dev = self.block_size, self.device
        N = b0 * bs
        bounds = kernels.head_chunks(R)
        n_sub = len(bounds)
        packed, qscale, qmin = self._quant(entries)
        sel = torch.empty((G, R, b0), dtype=torch.int32, device=dev)
        logits = torch.empty((G, R, N), dtype=torch.float32, device=dev)
        desired = torch.empty((G, R), dtype=torch.int32, device=dev)
        allocated = torch.empty((G, R), dtype=torch.int32, device=dev)
        head_bits = torch.empty((G, R, (N + 31) // 32), dtype=torch.int32, device=dev)
        sub_rows, sub_counts = [], []
        for r0, r1 in bounds:
            qs = q[:, r0:r1].contiguous()
            width = min(pmin.shape[1], (r1 - r0) * b0)
            sel_s = torch.empty((G, r1 - r0, b0), dtype=torch.int32, device=dev)
            plan_pages = torch.empty((G, width), dtype=torch.int32, device=dev)
            plan_masks = torch.empty((G, width), dtype=torch.uint8, device=dev)
            plan_counts = torch.empty((G,), dtype=torch.int32, device=dev)
            kernels.quest_select(qs, pmin, pmax, b0, sel_pages=sel_s, plan_pages=plan_pages, plan_masks=plan_masks,
                                 plan_counts=plan_counts)
            lg = kernels.twilight_qk(qs, packed, qscale, qmin, plan_pages, plan_masks, plan_counts, b0,
                                     sink=self.sink_tokens, block_size=bs)
            sel[:, r0:r1] = sel_s
            logits[:, r0:r1] = lg
            rows_s = torch.empty((G, old_length + 1), dtype=torch.int32, device=dev)
            counts_s = torch.empty((G,), dtype=torch.int32, device=dev)
            des_s = torch.empty((G, r1 - r0), dtype=torch.int32, device=dev)
            bits_s = torch.empty((G, r1 - r0, (N + 31) // 32), dtype=torch.int32, device=dev)
            kernels.twilight_select(lg, sel_s, top_p=self.top_p, budget_mode="dynamic", rows=rows_s,
                                    row_counts=counts_s, desired=des_s, head_bits=bits_s, sink=self.sink_tokens,
                                    recent=self.recent_tokens, block_size=bs, length=old_length)
            desired[:, r0:r1] = des_s
            head_bits[:, r0:r1] = bits_s
            sub_rows.append(rows_s)
            sub_counts.append(counts_s)
        if self.budget_mode == "matched":
            des_host = desired.cpu().tolist()
            alloc = [matched_budget_counts(d, fixed * bs * R, [N] * R) for d in des_host]
            allocated.copy_(torch.tensor(alloc, dtype=torch.int32))
            sub_rows, sub_counts = [], []
            for r0, r1 in bounds:
                rows_s = torch.empty((G, old_length + 1), dtype=torch.int32, device=dev)
                counts_s = torch.empty((G,), dtype=torch.int32, device=dev)
                bits_s = torch.empty((G, r1 - r0, (N + 31) // 32), dtype=torch.int32, device=dev)
                kernels.twilight_select(logits[:, r0:r1].contiguous(), sel[:, r0:r1].contiguous(), top_p=self.top_p,
                                        budget_mode="given", rows=rows_s, row_counts=counts_s,
                                        allocated=allocated[:, r0:r1].contiguous(), head_bits=bits_s,
                                        sink=self.sink_tokens, recent=self.recent_tokens, block_size=bs,
                                        length=old_length)
                head_bits[:, r0:r1] = bits_s
                sub_rows.append(rows_s)
                sub_counts.append(counts_s)
        else:
            allocated.copy_(desired)
        rows = torch.empty((G, old_length + 1), dtype=torch.int32, device=dev)
        counts = torch.empty((G,), dtype=torch.int32, device=dev)
        counts_host = torch.stack(sub_counts).cpu()
        for g in range(G):
            merged = torch.unique(torch.cat([sub_rows[i][g, :int(counts_host[i, g])] for i in range(n_sub)]))
            rows[g, :merged.numel()] = merged
            counts[g] = merged.numel()
        return dict(desired=desired, allocated=allocated, head_bits=head_bits, pages=sel, logits=logits, rows=rows,
                    counts=counts)

    def _quant(self, entries: Sequence[int]) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        assert self._packed is not None and self._qscale is not None and self._qmin is not None
        if self._consecutive(entries):
            e0, G = entries[0], len(entries)
            return self._packed[e0:e0 + G], self._qscale[e0:e0 + G], self._qmin[e0:e0 + G]
        idx = torch.tensor(list(entries), device=self.device)
        return self._packed[idx], self._qscale[idx], self._qmin[idx]

    def prepare_layer_selection(self, *, entries: list[int], queries: list[torch.Tensor]) -> None:
        """Both Twilight selection stages for every query head of a layer
        (twilight_offload_cache.py:996-1843); the result stays on the device
        for update_layer_gqa_group_ragged / update."""
        if not self.layer_batched_selection:
            return
        q = self._check_layer_queries(entries, queries)
        old_length = self._uniform_length(entries)
        state = self._select_layer(entries, q, old_length)
        for g, entry in enumerate(entries):
            self._prepared_layer[entry] = (state, g)
        self._trace_layer(state)

    def _layer_state(self, entries: Sequence[int], queries: Sequence[torch.Tensor], old_length: int) -> dict:
        prepared = [self._prepared_layer.pop(e, None) for e in entries]
        if all(p is not None for p in prepared):
            states = {id(p[0]) for p in prepared}
            if len(states) == 1 and [p[1] for p in prepared] == list(range(len(entries))):
                return prepared[0][0]
        q = torch.stack([query[0, :, 0] for query in queries], dim=0).float().contiguous()
        state = self._select_layer(entries, q, old_length)
        self._trace_layer(state)
        return state

    # ------------------------------------------------------------ GQA union
    def update_layer_gqa_group_ragged(
        self,
        *,
        key_states: list[torch.Tensor],
        value_states: list[torch.Tensor],
        queries: list[torch.Tensor],
        entries: list[int],
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, int, tuple[int, ...]]:
        """One shared union per KV group: (K[sum U_g + G, 1, D], V,
        cu_seqlens_k int32 [G+1] on the device, max_seqlen_k, lengths) where
        group g's segment is its union of the R heads' selections, the sink
        and the recent window, ascending, then the decode token
        (twilight_offload_cache.py:2610-3602).  The union rows are gathered
        on the device; one 4(G+1)-byte copy to the host gives the lengths."""
        if not self.gqa_groupwise_execution:
            raise RuntimeError("Twilight GQA group-wise execution is disabled")
        old_length = self._advance_layer(entries, key_states, value_states, queries)
        self._wait_host_writes(entries)
        state = self._layer_state(entries, queries, old_length)
        G, D = len(entries), self.geometry.head_dim
        cap = G * (old_length + 1)
        if self._flat_union_keys is None or self._flat_union_keys.shape[0] < cap:
            self._flat_union_keys = torch.empty((cap, 1, D), dtype=self.dtype, device=self.device)
            self._flat_union_values = torch.empty_like(self._flat_union_keys)
        assert self._flat_union_values is not None
        cur_k = torch.cat([k[0, 0] for k in key_states], dim=0).contiguous()
        cur_v = torch.cat([v[0, 0] for v in value_states], dim=0).contiguous()
        cu = torch.empty((G + 1,), dtype=torch.int32, device=self.device)
        flat_k, flat_v = self._flat_union_keys, self._flat_union_values
        start = self._phase_start()
        if self.post_selection_pipeline and self.kv_residency == "host":
            cu_host = self._pipelined_union_gather(entries, state, cur_k, cur_v)
            cu.copy_(cu_host.to(torch.int32), non_blocking=True)
        elif self._consecutive(entries):
            resident = None
            if self.previous_token_resident_cache and self.kv_residency == "host":
                flat_k, flat_v, cu, resident = self._gqa_resident_buffers(entries, old_length)
            kernels.gather_union(self._key_rows, self._value_rows, state["rows"], state["counts"], cur_k, cur_v,
                                 flat_k.view(-1, D), flat_v.view(-1, D), cu,
                                 entry_row0=self.geometry.row(entries[0], 0),
                                 entry_row_step=self.geometry.max_cache_len, max_count=state["max_count"],
                                 error_flag=self._gather_error, resident=resident)
        else:
            raise ValueError("GQA group execution needs the consecutive entries of one layer")
        self._phase_end("gather", start)
        self._append(entries, cur_k, cur_v, old_length)
        if not (self.post_selection_pipeline and self.kv_residency == "host"):
            cu_host = cu.cpu()
        lengths = tuple(int(cu_host[g + 1] - cu_host[g]) for g in range(G))
        total = int(cu_host[-1])
        for g, entry in enumerate(entries):
            self._last_query_head_lengths[entry] = (lengths[g],) * self.num_query_heads_per_kv
        if self.metrics_enabled:
            self.metrics["cache_update_calls"] += 1
            self.metrics["attention_valid_tokens_total"] += total
            self.metrics["gather_bytes"] += 2 * (total - G) * D * cur_k.element_size()
        return flat_k[:total], flat_v[:total], cu, max(lengths), lengths

    def _gqa_resident_buffers(self, entries: Sequence[int], old_length: int):
        """This layer's packed-union buffers of the resident GQA-group path: two
        alternating by the length's parity (this step packs into one while the
        previous step's stays readable), their cu_seqlens, the position map
        and the stats; the gather's resident arguments."""
        G, D = len(entries), self.geometry.head_dim
        layer = entries[0] // G
        st = self._gqa_resident.get(layer)
        if st is None:
            R = self.num_query_heads_per_kv
            b0 = max(1, math.ceil(self.candidate_token_budget / self.block_size))
            per_group = min(self.geometry.max_cache_len,
                            self.sink_tokens + R * b0 * self.block_size + self.recent_tokens) + 1
            cap = G * per_group
            st = {"k": [torch.empty((cap, 1, D), dtype=self.dtype, device=self.device) for _ in range(2)],
                  "v": [torch.empty((cap, 1, D), dtype=self.dtype, device=self.device) for _ in range(2)],
                  "cu": [torch.zeros((G + 1,), dtype=torch.int32, device=self.device) for _ in range(2)],
                  "map": torch.full((G, self.geometry.max_cache_len), -1, dtype=torch.int64, device=self.device),
                  "stats": torch.zeros((2,), dtype=torch.int64, device=self.device)}
            self._gqa_resident[layer] = st
        par = old_length & 1
        resident = dict(map=st["map"], epoch=old_length, prev_k=st["k"][1 - par].view(-1, D),
                        prev_v=st["v"][1 - par].view(-1, D), prev_cu=st["cu"][1 - par], stats=st["stats"])
        return st["k"][par], st["v"][par], st["cu"][par], resident

    def resident_stats(self) -> dict[str, int]:
        """Rows read from the HBM resident cache vs. all union rows, over the
        fused decode and the GQA-group path (cumulative; synchronizes the
        device).  The keys are the Quest cache's, whose counts are pages."""
        out = super().resident_stats()
        hits, rows = out["resident_hit_pages"], out["union_pages"]
        for st in self._gqa_resident.values():
            h, r = st["stats"].tolist()
            hits, rows = hits + int(h), rows + int(r)
        return {"resident_hit_pages": hits, "union_pages": rows}

    # ------------------------------------------------------------ fast path
    def decode_layer(self, *, queries: torch.Tensor, key_states: torch.Tensor, value_states: torch.Tensor,
                     entries: Sequence[int], softmax_scale: Optional[float] = None,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """One decoder layer's Twilight decode with no host sync: both
        selection stages and the GQA union on the device (Quest B0, INT4 QK,
        top-p, union rows), then the split-K attention reading the union rows
        and the decode token straight from the slab, with the append fused.

        queries [G, R, D] in the cache dtype; key_states/value_states [G, D];
        entries consecutive.  Returns [G, R, D]."""
        G, R, D = queries.shape
        if R != self.num_query_heads_per_kv or D != self.geometry.head_dim or len(entries) != G:
            raise ValueError("queries must be [len(entries), num_query_heads_per_kv, head_dim]")
        if key_states.shape != (G, D) or value_states.shape != (G, D):
            raise ValueError("key_states/value_states must be [G, head_dim]")
        if not self._consecutive(entries):
            raise ValueError("decode_layer needs the consecutive entries of one layer")
        for e in entries:
            self._bookkeeping.advance(e, 1)
            self._initialized[e] = True
        self._seen_tokens = self._bookkeeping.seen_tokens
        old_length = self._logical_lengths[entries[0]] - 1
        self._wait_host_writes(entries)
        fused = self._decode_layer_fused(queries, key_states, value_states, entries, old_length, softmax_scale, out)
        if fused is not None:
            return fused
        state = self._select_layer(entries, queries.float().contiguous(), old_length)
        self._trace_layer(state)
        e0 = entries[0]
        cur_k, cur_v = key_states.contiguous(), value_states.contiguous()
        start = self._phase_start()
        # the union rows are below old_length, so the decode token's row is
        # written by the attention launch itself
        result = kernels.decode_attention_rows(queries.contiguous(), self._key_cache[e0:e0 + G],
                                               self._value_cache[e0:e0 + G], state["rows"], state["counts"],
                                               state["max_count"], cur_k=cur_k, cur_v=cur_v,
                                               softmax_scale=softmax_scale, out=out, append_position=old_length)
        self._phase_end("attention", start)
        self._append(entries, cur_k, cur_v, old_length, written=True)
        for e in entries:
            self._last_query_head_lengths[e] = None
        return result

    def _decode_layer_fused(self, queries: torch.Tensor, key_states: torch.Tensor, value_states: torch.Tensor,
                            entries: Sequence[int], old_length: int, softmax_scale: Optional[float],
                            out: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
        """decode_layer through the fused selection: the Quest score and the
        INT4 QK of every scored row, then per (group, head) the B0 top-k and
        top-p into the group's union record (matched budgets: the top-p
        counts, then the group's allocation and each head's top-allocated
        rows in one more launch), and the attention over the record's kept
        rows (the same token set as the union row list).  More than 8 query
        heads per KV head run as sub-groups (with matched budgets, up to 64
        heads sharing one allocation).  None when the layer takes the general
        path: other shapes, matched budgets over more than 64 heads, or traces
        that record the row list."""
        G, R, D = queries.shape
        # more than 8 query heads per KV head run as sub-groups; one wavefront
        # forms a matched allocation, a lane a head
        if (not self.fused_decode or (R > 64 and self.budget_mode == "matched") or D != 128 or self.block_size != 16
                or self.dtype not in (torch.float16, torch.bfloat16) or self._capture_selection_trace
                or self._capture_budget_trace or self._page_min is None or self._packed is None):
            return None
        sink_end, recent_start, cand, fixed, b0 = self._twilight_budgets(old_length)
        if cand == 0 or fixed == 0 or b0 == 0 or cand > 8192 or b0 * self.block_size > 8192:
            return None
        matched = self.budget_mode == "matched"
        if matched and fixed > b0:  # a target past every candidate: the general path reports it
            return None
        pmin, pmax = self._metadata(entries, cand)
        packed, qscale, qmin = self._quant(entries)
        if packed.shape[1] < self.sink_tokens + cand * self.block_size:
            return None
        # one record row per group, sized for every page of the metadata (the
        # entry points take any row stride that is a multiple of 4 words), and
        # the counts: allocated once, reused by every layer in stream order
        if self._fused_bufs is None or self._fused_bufs[0].shape[0] != G or self._fused_bufs[1].shape[1] != R:
            words = (kernels.union_record_words(int(self._page_min.shape[1])) + 3) & ~3
            self._fused_bufs = (torch.empty((G, words), dtype=torch.int32, device=self.device),
                                torch.empty((G, R), dtype=torch.int32, device=self.device))
        rec, desired = self._fused_bufs
        start = self._phase_start()
        kernels.twilight_select_fused(queries.float().contiguous(), pmin, pmax, packed, qscale, qmin, b0, rec,
                                      top_p=self.top_p, sink=self.sink_tokens, recent=self.recent_tokens,
                                      block_size=self.block_size, length=old_length, desired=desired,
                                      budget_mode=self.budget_mode,
                                      target_total=fixed * self.block_size * R if matched else 0)
        self._phase_end("twilight_fused_selection", start)
        e0 = entries[0]
        cur_k, cur_v = key_states.contiguous(), value_states.contiguous()
        start = self._phase_start()
        resident = self.resident_pages().view(e0, G) if self._resident_active else None
        result = kernels.decode_attention_union(queries.contiguous(), self._key_cache[e0:e0 + G],
                                                self._value_cache[e0:e0 + G], rec, cand,
                                                max_pages=min(cand, R * b0), sink=self.sink_tokens,
                                                recent=self.recent_tokens, block_size=self.block_size,
                                                length=old_length, append=True, cur_k=cur_k, cur_v=cur_v,
                                                softmax_scale=softmax_scale, out=out, resident=resident)
        self._phase_end("attention", start)
        self._append(entries, cur_k, cur_v, old_length, written=True)
        for e in entries:
            self._last_query_head_lengths[e] = None
        return result

    # ----------------------------------------------------- per-head selection
    def _head_positions(self, state: dict, g: int) -> list[torch.Tensor]:
        """Each head's own selected positions (sink ++ kept candidates ++
        recent, ascending) for group g of a layer state, on the device."""
        old_length = state["old_length"]
        sink_end, recent_start, _ = _window(old_length, self.sink_tokens, self.recent_tokens)
        dev = self.device
        sink = torch.arange(sink_end, device=dev, dtype=torch.int64)
        recent = torch.arange(recent_start, old_length, device=dev, dtype=torch.int64)
        R = self.num_query_heads_per_kv
        if state["pages"] is None:
            return [torch.cat([sink, recent]) for _ in range(R)]
        pages = state["pages"][g].to(torch.int64)                       # [R, b0]
        bs = self.block_size
        cand = (self.sink_tokens + pages[:, :, None] * bs + torch.arange(bs, device=dev)).reshape(R, -1)
        N = cand.shape[1]
        words = state["head_bits"][g].to(torch.int64) & 0xFFFFFFFF     # [R, W]
        bit = (words[:, :, None] >> torch.arange(32, device=dev)) & 1
        keep = bit.reshape(R, -1)[:, :N].bool()
        return [torch.cat([sink, cand[r][keep[r]], recent]) for r in range(R)]

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: Optional[Dict[str, Any]] = None):
        """Per-entry decode with each query head's own Twilight selection
        (twilight_offload_cache.py:1845-2051), packed [1, R, Tmax, D]; prefill
        as in the Quest cache."""
        if key_states.shape[-2] > 1 or key_states.shape[:2] != (1, 1):
            return super().update(key_states, value_states, layer_idx, cache_kwargs)
        query = None if cache_kwargs is None else cache_kwargs.get("query_states")
        R, D = self.num_query_heads_per_kv, self.geometry.head_dim
        if key_states.shape != value_states.shape or key_states.shape[-1] != D or key_states.dtype != self.dtype:
            raise ValueError("expected identical head-wise [1, 1, seq, dim] K/V")
        if query is None or tuple(query.shape) != (1, R, 1, D):
            raise ValueError("decode requires post-RoPE query_states")
        old_length, _ = self._bookkeeping.advance(layer_idx, 1)
        self._seen_tokens = self._bookkeeping.seen_tokens
        self._initialized[layer_idx] = True
        self._wait_host_writes([layer_idx])
        prepared = self._prepared_layer.pop(layer_idx, None)
        if prepared is not None:
            state, g = prepared
        else:
            state = self._select_layer([layer_idx], query[0, :, 0].float().unsqueeze(0).contiguous(), old_length)
            g = 0
            self._trace_layer(state)
        positions = self._head_positions(state, g)
        lengths = [int(p.numel()) for p in positions]
        total = max(lengths) + 1
        self._ensure_pack(total)
        row0 = self.geometry.row(layer_idx, 0)
        src = torch.cat([p + row0 for p in positions])
        dst = torch.cat([torch.arange(n, device=self.device, dtype=torch.int64) * R + r
                         for r, n in enumerate(lengths)])
        kernels.gather_rows(self._key_rows, self._value_rows, src, self._pack_rows_k, self._pack_rows_v, dst,
                            error_flag=self._gather_error)
        cur_k = key_states[0, 0].contiguous()
        cur_v = value_states[0, 0].contiguous()
        for r, n in enumerate(lengths):
            self._pack_rows_k[n * R + r].copy_(cur_k[0])
            self._pack_rows_v[n * R + r].copy_(cur_v[0])
        self._append([layer_idx], cur_k, cur_v, old_length)
        self._last_query_head_lengths[layer_idx] = tuple(n + 1 for n in lengths)
        assert self._gpu_pack_keys is not None and self._gpu_pack_values is not None
        return (self._gpu_pack_keys[:, :total].transpose(1, 2), self._gpu_pack_values[:, :total].transpose(1, 2))

    def update_layer_flat_ragged(
        self,
        *,
        key_states: list[torch.Tensor],
        value_states: list[torch.Tensor],
        queries: list[torch.Tensor],
        entries: list[int],
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, int, tuple[int, ...]]:
        """Every query head's own Twilight selection as one ragged batch
        (segment (g, r) = head r's positions ++ the decode token), the
        layer-flat form of quest_offload_cache.py:724-987."""
        if not self.layer_flat_ragged_execution:
            raise RuntimeError("layer-flat ragged execution is disabled")
        old_length = self._advance_layer(entries, key_states, value_states, queries)
        self._wait_host_writes(entries)
        state = self._layer_state(entries, queries, old_length)
        D, dev = self.geometry.head_dim, self.device
        srcs, dsts, tok_rows, tok_src, lengths = [], [], [], [], []
        off = 0
        for g, entry in enumerate(entries):
            row0 = self.geometry.row(entry, 0)
            for pos in self._head_positions(state, g):
                n = int(pos.numel())
                srcs.append(pos + row0)
                dsts.append(torch.arange(off, off + n, device=dev, dtype=torch.int64))
                tok_rows.append(off + n)
                tok_src.append(g)
                lengths.append(n + 1)
                off += n + 1
        if self._flat_keys is None or self._flat_keys.shape[0] < off:
            self._flat_keys = torch.empty((off, 1, D), dtype=self.dtype, device=dev)
            self._flat_values = torch.empty_like(self._flat_keys)
        assert self._flat_values is not None
        fk, fv = self._flat_keys.view(-1, D), self._flat_values.view(-1, D)
        kernels.gather_rows(self._key_rows, self._value_rows, torch.cat(srcs), fk, fv, torch.cat(dsts),
                            error_flag=self._gather_error)
        cur_k = torch.cat([k[0, 0] for k in key_states], dim=0).contiguous()
        cur_v = torch.cat([v[0, 0] for v in value_states], dim=0).contiguous()
        rows = torch.tensor(tok_rows, device=dev)
        srcg = torch.tensor(tok_src, device=dev)
        fk.index_copy_(0, rows, cur_k.index_select(0, srcg))
        fv.index_copy_(0, rows, cur_v.index_select(0, srcg))
        self._append(entries, cur_k, cur_v, old_length)
        R = self.num_query_heads_per_kv
        for g, entry in enumerate(entries):
            self._last_query_head_lengths[entry] = tuple(lengths[g * R:(g + 1) * R])
        cu = torch.tensor([0, *torch.tensor(lengths).cumsum(0).tolist()], dtype=torch.int32, device=dev)
        return self._flat_keys[:off], self._flat_values[:off], cu, max(lengths), tuple(lengths)

    def _pipelined_union_gather(self, entries: Sequence[int], state: dict, cur_k: torch.Tensor,
                                cur_v: torch.Tensor) -> torch.Tensor:
        """The union rows of every group through the side-stream DMA pipeline
        (the reference's post_selection_pipeline, twilight_offload_cache.py:
        2053-2455): the union row lists come to the host once, then every
        chunk of post_selection_groups_per_chunk groups is gathered on the CPU
        from the pinned slab and copied to the flat attention layout on the
        pipeline's stream while the next chunk is gathered.  Each group's gap
        row takes its decode token on the device afterwards.  Returns the
        cu_seqlens on the host."""
        import numpy as np

        from .dma_pipeline import HostGatherPipeline

        G, D = len(entries), self.geometry.head_dim
        counts = state["counts"].cpu().numpy().astype(np.int64)
        rows = state["rows"][:, :max(1, int(counts.max()) if G else 1)].cpu().numpy().astype(np.int64)
        cu = np.concatenate([[0], np.cumsum(counts + 1)])
        per = max(1, self.post_selection_groups_per_chunk)
        fk = self._flat_union_keys.view(-1, D)
        fv = self._flat_union_values.view(-1, D)
        chunks = []
        for c0 in range(0, G, per):
            gs = range(c0, min(G, c0 + per))
            # each group's rows, then a placeholder for its decode token's row
            ids = np.concatenate([np.append(self.geometry.row(entries[g], 0) + rows[g, :counts[g]], 0) for g in gs])
            a, b = int(cu[c0]), int(cu[gs[-1] + 1])
            chunks.append((ids, fk[a:b], fv[a:b]))
        need = max(int(c[0].shape[0]) for c in chunks) if chunks else 1
        if self._dma is None or self._dma.max_rows < need:
            self._dma = HostGatherPipeline(self.device, D, self.dtype, need)
        self._dma.run(self._key_rows, self._value_rows, chunks)
        gap = torch.from_numpy(cu[1:] - 1).to(self.device)
        fk.index_copy_(0, gap, cur_k)
        fv.index_copy_(0, gap, cur_v)
        return torch.from_numpy(cu)

    # ----------------------------------------------------------------- traces
    def enable_budget_trace(self, enabled: bool = True) -> None:
        self._capture_budget_trace = bool(enabled)
        self._budget_trace = []

    def budget_trace(self) -> list[dict[str, Any]]:
        return list(self._budget_trace)

    def group_union_trace(self) -> list[dict[str, Any]]:
        return list(self._group_union_trace)

    def _trace_layer(self, state: dict) -> None:
        if not (self._capture_selection_trace or self._capture_budget_trace):
            return
        old_length = state["old_length"]
        decode_step = old_length - self._prompt_length + 1 if self._prompt_length is not None else None
        counts = state["counts"].cpu()
        rows = state["rows"].cpu()
        desired = None if state["desired"] is None else state["desired"].cpu()
        allocated = None if state["allocated"] is None else state["allocated"].cpu()
        for g, entry in enumerate(state["entries"]):
            if self._capture_budget_trace:
                self._budget_trace.append({
                    "decode_step": decode_step, "entry": entry, "b0_pages": state["b0"],
                    "fixed_pages": state["fixed"],
                    "desired": None if desired is None else tuple(int(v) for v in desired[g]),
                    "allocated": None if allocated is None else tuple(int(v) for v in allocated[g])})
            if self._capture_selection_trace:
                union = rows[g, :int(counts[g])]
                self._group_union_trace.append({
                    "decode_step": decode_step, "entry": entry, "group_tokens": int(union.numel()),
                    "positions_sha256": hashlib.sha256(union.to(torch.int64).numpy().tobytes()).hexdigest()})
                for r, pos in enumerate(self._head_positions(state, g)):
                    self._selection_trace.append({
                        "decode_step": decode_step, "entry": entry, "query_head_in_group": r,
                        "selected_positions_sha256": hashlib.sha256(pos.cpu().numpy().tobytes()).hexdigest(),
                        "selected_tokens": int(pos.numel())})

    def selected_positions_sha256(self) -> str:
        digest = hashlib.sha256()
        for item in self._selection_trace:
            digest.update(repr(sorted(item.items())).encode())
        return digest.hexdigest()

    def group_positions_sha256(self) -> Optional[str]:
        if not self._group_union_trace:
            return None
        digest = hashlib.sha256()
        for item in self._group_union_trace:
            digest.update(repr(sorted(item.items())).encode())
        return digest.hexdigest()

    def state_snapshot(self) -> Dict[str, Any]:
        snap = super().state_snapshot()
        quant = sum(t.numel() * t.element_size() for t in (self._packed, self._qscale, self._qmin) if t is not None)
        snap.update({
            "policy": ("twilight_int4_top_p_dynamic" if self.budget_mode == "dynamic"
                       else "twilight_int4_top_p_matched_quest"),
            "candidate_token_budget": self.candidate_token_budget,
            "top_p": self.top_p,
            "matched_budget_fraction": self.matched_budget_fraction,
            "budget_mode": self.budget_mode,
            "quantized_key_metadata_gpu_bytes": quant,
            "twilight_gqa_groupwise_execution": self.gqa_groupwise_execution,
            "layer_batched_twilight_selection": self.layer_batched_selection,
            "selection_device": "gpu (tw_quest_select, tw_twilight_qk, tw_twilight_select)",
            "twilight_gqa_group_semantics": "exact union of the original per-Query-head selected token sets",
            **{f"requested_{k}": v for k, v in self._variant_flags.items()},
        })
        return snap
