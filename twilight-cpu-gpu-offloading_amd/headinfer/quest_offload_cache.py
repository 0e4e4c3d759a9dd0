"""Quest-style per-query-head sparse decode cache on one MI355X.

Call surface of QuestTopKOffloadedCache (quest_offload_cache.py:22-1055):
the constructor keywords and defaults, ``from_llama_model``, ``update``,
``prepare_layer_selection``, ``update_layer_flat_ragged``,
``get_last_query_head_lengths``, the lifecycle methods, metrics and the
selection trace.  Selection semantics are the reference's: per query head a
fixed budget of k pages ranked by the Quest upper bound over the KV head's
page min/max metadata (ties to the lowest page), plus the sink and recent
windows and the decode token.

What differs is where the work runs.  The reference scores on the GPU,
synchronizes the page ids to the CPU, gathers the rows with index_select into
pinned staging and copies them to the GPU.  Here the selection never leaves
the GPU: tw_quest_select writes the page ids (and the GQA union plan) on the
device, the gather kernels read the selected rows straight out of the slab
-- HBM, or pinned host memory through its mapped device address (zero-copy
over the host link) -- and the decode token is appended to the slab by a
kernel on the same stream.  ``decode_layer`` is the one-call fast path:
selection plus the sparse attention that reads the union pages directly from
the slab, with the append fused into the attention launch.

Storage: one slab [2, entries, max_cache_len, head_dim] (K plane, then V),
pinned host memory (``kv_residency="host"``, the reference's layout) or HBM
(``"hbm"``).  Page metadata [entries, prompt_pages, head_dim] and all
selection state live in HBM.
"""

from __future__ import annotations

import math
import time
from collections import defaultdict
from typing import Any, Dict, Optional, Sequence, Tuple

import torch

from . import kernels
from .slab_cache import SequentialCacheState, SlabGeometry

try:  # the reference caches are transformers Cache objects
    from transformers.cache_utils import Cache as _HFCache
except Exception:  # pragma: no cover - transformers is optional
    _HFCache = object

__all__ = ["QuestTopKOffloadedCache"]


class _CacheBase(_HFCache):  # type: ignore[misc, valid-type]
    def __init__(self) -> None:
        if _HFCache is object:
            return
        try:
            super().__init__(layers=[])
        except TypeError:  # older transformers: no-argument Cache
            super().__init__()


def _window(length: int, sink: int, recent: int) -> tuple[int, int, int]:
    """(sink_end, recent_start, eligible) of quest_offload_cache.py:326-333."""
    sink_end = min(sink, length)
    recent_start = max(sink_end, length - max(0, recent - 1))
    return sink_end, recent_start, max(0, recent_start - sink_end)


class QuestTopKOffloadedCache(_CacheBase):
    """Slab-backed KV cache with per-query-head Quest top-k page selection."""

    def __init__(
        self,
        *,
        num_cache_entries: int,
        max_cache_len: int,
        head_dim: int,
        num_query_heads_per_kv: int,
        dtype: torch.dtype,
        device: torch.device | str,
        sink_tokens: int = 64,
        recent_tokens: int = 256,
        block_size: int = 16,
        budget_fraction: float = 0.05,
        selection_interval: int = 1,
        max_selected_history_fraction: Optional[float] = None,
        layer_batched_selection: bool = False,
        layer_flat_ragged_execution: bool = False,
        sparse_gather_stabilized: bool = False,
        per_head_varlen_attention_reference: bool = False,
        kv_residency: str = "host",
        budget_pages: Optional[int] = None,
        update_metadata_on_decode: bool = False,
        previous_token_resident_cache: bool = False,
    ) -> None:
        super().__init__()
        device = torch.device(device)
        if device.type != "cuda" or not torch.cuda.is_available():
            raise ValueError("an operational ROCm device is required")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        if sink_tokens < 0 or recent_tokens <= 0 or block_size <= 0:
            raise ValueError("invalid sink/recent/block configuration")
        if not 0.0 < budget_fraction <= 1.0:
            raise ValueError("budget_fraction must be in (0, 1]")
        if selection_interval <= 0:
            raise ValueError("selection_interval must be positive")
        if max_selected_history_fraction is None:
            max_selected_history_fraction = budget_fraction
        if not 0.0 < max_selected_history_fraction <= 1.0:
            raise ValueError("max_selected_history_fraction must be in (0, 1]")
        if num_query_heads_per_kv <= 0:
            raise ValueError("num_query_heads_per_kv must be positive")
        if layer_flat_ragged_execution and not layer_batched_selection:
            raise ValueError("layer-flat ragged execution requires layer-batched selection")
        if sparse_gather_stabilized and not layer_flat_ragged_execution:
            raise ValueError("stabilized sparse gather requires layer-flat ragged execution")
        if kv_residency not in ("host", "hbm"):
            raise ValueError("kv_residency must be 'host' or 'hbm'")
        if budget_pages is not None and budget_pages <= 0:
            raise ValueError("budget_pages must be positive")
        if dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError("dtype must be float16, bfloat16 or float32")

        self.geometry = SlabGeometry(num_entries=num_cache_entries, batch_size=1, max_cache_len=max_cache_len,
                                     head_dim=head_dim)
        self.dtype = dtype
        self.device = device
        self.allocated_capacity = max_cache_len
        self.num_query_heads_per_kv = num_query_heads_per_kv
        self.sink_tokens = sink_tokens
        self.recent_tokens = recent_tokens
        self.block_size = block_size
        self.budget_fraction = budget_fraction
        self.budget_pages = budget_pages
        self.selection_interval = int(selection_interval)
        self.max_selected_history_fraction = max_selected_history_fraction
        self.layer_batched_selection = bool(layer_batched_selection)
        self.layer_flat_ragged_execution = bool(layer_flat_ragged_execution)
        self.sparse_gather_stabilized = bool(sparse_gather_stabilized)
        self.per_head_varlen_attention_reference = bool(per_head_varlen_attention_reference)
        self.kv_residency = kv_residency
        # The reference builds page metadata at prefill only and caps the
        # candidate pages at the prompt's; with this flag every decode append
        # also writes the new row's metadata (pages completed during decode
        # become candidates).
        self.update_metadata_on_decode = bool(update_metadata_on_decode)
        # The reference's previous-token resident cache (twilight_offload_cache.py:2457-2608): union pages
        # stay in an HBM page cache and only the pages the previous step did not read cross the host link.
        self.previous_token_resident_cache = bool(previous_token_resident_cache)
        if self.previous_token_resident_cache and (kv_residency != "host" or block_size != 16 or head_dim != 128
                                                   or dtype == torch.float32 or num_query_heads_per_kv > 8):
            raise ValueError("the resident page cache serves a host slab of 16-bit K/V, head_dim 128, 16-row pages "
                             "and at most 8 query heads per KV head")
        self._resident: Optional[kernels.ResidentPages] = None

        self._bookkeeping = SequentialCacheState(num_cache_entries, max_cache_len)
        self._logical_lengths = self._bookkeeping.logical_lengths
        self._initialized = [False] * num_cache_entries
        self._seen_tokens = 0

        E, L, D = num_cache_entries, max_cache_len, head_dim
        if kv_residency == "host":
            self._slab = torch.empty(self.geometry.total_elements, dtype=dtype, device="cpu", pin_memory=True)
        else:
            self._slab = torch.empty(self.geometry.total_elements, dtype=dtype, device=device)
        planes = self._slab.view(2, E, L, D)
        self._key_cache = planes[0]          # [E, Lmax, D]
        self._value_cache = planes[1]
        self._key_rows = planes[0].view(-1, D)
        self._value_rows = planes[1].view(-1, D)

        max_pages = math.ceil(max(0, max_cache_len - sink_tokens) / block_size)
        budget_cap = (budget_pages if budget_pages is not None
                      else max(1, math.ceil(max_selected_history_fraction * max_pages)))
        self.max_selected_tokens_per_query_head = min(max_cache_len,
                                                      sink_tokens + recent_tokens + budget_cap * block_size)
        self._gpu_pack_keys: Optional[torch.Tensor] = None
        self._gpu_pack_values: Optional[torch.Tensor] = None
        self._flat_keys: Optional[torch.Tensor] = None
        self._flat_values: Optional[torch.Tensor] = None
        self._layer_flat_group_count: Optional[int] = None

        self.eviction_stream = torch.cuda.Stream(device=device)
        # Set by a gather kernel that met a row outside the slab or its
        # destination (the row is skipped); synchronize() raises on it, so the
        # decode path itself needs no host sync to report a bad index.
        self._gather_error = torch.zeros(1, dtype=torch.int32, device=device)
        self._host_write_done: list[Optional[torch.cuda.Event]] = [None] * E
        self._page_min: Optional[torch.Tensor] = None   # [E, prompt_pages, D]
        self._page_max: Optional[torch.Tensor] = None
        self._prompt_length: Optional[int] = None
        self._last_query_head_lengths: list[Optional[tuple[int, ...]]] = [None] * E
        self._cached_selected_pages: list[Optional[torch.Tensor]] = [None] * E   # [1, R, k] int32 device
        self._layer_prepared_entries: set[int] = set()
        self._capture_selection_trace = False
        self._selection_trace: list[dict[str, Any]] = []

        self.metrics_enabled = False
        self.metrics: Dict[str, float] = defaultdict(float)
        self._timing_events: list[tuple[str, torch.cuda.Event, torch.cuda.Event]] = []

    # ------------------------------------------------------------ construction
    @classmethod
    def from_llama_model(cls, model: torch.nn.Module, **kwargs: Any) -> "QuestTopKOffloadedCache":
        """Size the cache for a Llama-style model (quest_offload_cache.py:176-190)."""
        config = model.config
        parameter = next(model.parameters())
        return cls(
            num_cache_entries=config.num_hidden_layers * config.num_key_value_heads,
            head_dim=getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads,
            num_query_heads_per_kv=config.num_attention_heads // config.num_key_value_heads,
            dtype=parameter.dtype,
            device=parameter.device,
            **kwargs,
        )

    # ----------------------------------------------------------------- metrics
    def _stream(self) -> torch.cuda.Stream:
        return torch.cuda.current_stream(self.device)

    def reset_metrics(self) -> None:
        self.metrics = defaultdict(float)
        self._timing_events = []

    def enable_metrics(self, enabled: bool = True) -> None:
        self.metrics_enabled = bool(enabled)
        if enabled:
            self.reset_metrics()

    def _phase_start(self) -> Optional[torch.cuda.Event]:
        if not self.metrics_enabled:
            return None
        ev = torch.cuda.Event(enable_timing=True)
        ev.record(self._stream())
        return ev

    def _phase_end(self, name: str, start: Optional[torch.cuda.Event]) -> None:
        if start is None:
            return
        end = torch.cuda.Event(enable_timing=True)
        end.record(self._stream())
        self._timing_events.append((name, start, end))

    def resolve_metrics(self) -> Dict[str, float]:
        self.synchronize()
        for name, start, end in self._timing_events:
            self.metrics[f"{name}_cuda_seconds"] += start.elapsed_time(end) / 1000.0
            self.metrics[f"{name}_event_intervals"] += 1
        self._timing_events = []
        return dict(self.metrics)

    # ------------------------------------------------------------------ traces
    def enable_selection_trace(self, enabled: bool = True) -> None:
        """Record the selected page ids (a device-to-host copy per selection;
        for correctness runs only)."""
        self._capture_selection_trace = bool(enabled)
        self._selection_trace = []

    def selection_trace(self) -> list[dict[str, Any]]:
        return list(self._selection_trace)

    def _trace_selection(self, decode_step: int, entries: Sequence[int], sel: Optional[torch.Tensor]) -> None:
        if not self._capture_selection_trace:
            return
        host = None if sel is None else sel.cpu()
        for g, entry in enumerate(entries):
            for r in range(self.num_query_heads_per_kv):
                pages = () if host is None else tuple(int(v) for v in host[g, r].tolist())
                self._selection_trace.append({"decode_step": decode_step, "entry": entry, "query_head_in_group": r,
                                              "selected_page_indices": pages})

    # -------------------------------------------------------------- lifecycle
    def get_last_query_head_lengths(self, entry: int) -> Optional[tuple[int, ...]]:
        """Valid packed K/V length of each query head of an entry (history + decode token)."""
        return self._last_query_head_lengths[entry]

    def synchronize(self) -> None:
        self._stream().synchronize()
        self.eviction_stream.synchronize()
        if int(self._gather_error.item()):
            self._gather_error.zero_()
            raise RuntimeError("a K/V gather met a row index outside the slab or its destination")

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        return self._logical_lengths[0 if layer_idx is None else layer_idx]

    def get_max_length(self) -> Optional[int]:
        return self.allocated_capacity

    def get_max_cache_shape(self, layer_idx: int = 0) -> int:
        return self.allocated_capacity

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        del beam_idx
        raise NotImplementedError("batch-size-1 cache does not support reordering")

    def state_snapshot(self) -> Dict[str, Any]:
        def nbytes(*ts: Optional[torch.Tensor]) -> int:
            return sum(t.numel() * t.element_size() for t in ts if t is not None)

        return {
            "policy": "quest_topk_pages",
            "kv_residency": self.kv_residency,
            "num_cache_entries": self.geometry.num_entries,
            "max_cache_len": self.geometry.max_cache_len,
            "head_dim": self.geometry.head_dim,
            "num_query_heads_per_kv": self.num_query_heads_per_kv,
            "sink_tokens": self.sink_tokens,
            "recent_tokens": self.recent_tokens,
            "block_size": self.block_size,
            "budget_fraction": self.budget_fraction,
            "budget_pages": self.budget_pages,
            "selection_interval": self.selection_interval,
            "layer_batched_selection": self.layer_batched_selection,
            "layer_flat_ragged_execution": self.layer_flat_ragged_execution,
            "update_metadata_on_decode": self.update_metadata_on_decode,
            "previous_token_resident_cache": self.previous_token_resident_cache,
            "logical_lengths": list(self._logical_lengths),
            "seen_tokens": self._seen_tokens,
            "prompt_length": self._prompt_length,
            "slab_bytes": nbytes(self._slab),
            "metadata_gpu_bytes": nbytes(self._page_min, self._page_max),
            "execution_gpu_bytes": nbytes(self._gpu_pack_keys, self._gpu_pack_values, self._flat_keys,
                                          self._flat_values),
        }

    # ---------------------------------------------------------------- prefill
    def _build_metadata(self, entry: int, key_states: torch.Tensor) -> None:
        """Page min/max of the prompt's complete pages (quest_offload_cache.py:276-289)."""
        keys = key_states[0, 0]
        T = int(keys.shape[0])
        pages = (T - self.sink_tokens) // self.block_size if T > self.sink_tokens else 0
        if self._page_min is None:
            shape = (self.geometry.num_entries, self._metadata_page_capacity(pages), self.geometry.head_dim)
            self._page_min = torch.empty(shape, dtype=self.dtype, device=self.device)
            self._page_max = torch.empty(shape, dtype=self.dtype, device=self.device)
        if pages:
            kernels.build_page_metadata(keys.contiguous(), sink=self.sink_tokens, block_size=self.block_size,
                                        page_min=self._page_min[entry], page_max=self._page_max[entry])

    def _metadata_page_capacity(self, prompt_pages: int) -> int:
        if not self.update_metadata_on_decode:
            return max(prompt_pages, 0)
        return max(prompt_pages, (self.geometry.max_cache_len - self.sink_tokens) // self.block_size, 0)

    def _update_decode_metadata(self, entries: Sequence[int], position: int) -> None:
        """Metadata of the decode row `position` just appended to the entries
        (stream-ordered after the append): the page it completes, if any."""
        if not self.update_metadata_on_decode or self._page_min is None:
            return
        start = self._phase_start()
        for e0, n in self._runs(entries):
            kernels.update_page_metadata(self._key_cache, first_entry=e0, n_entries=n, position=position,
                                         sink=self.sink_tokens, block_size=self.block_size,
                                         page_min=self._page_min, page_max=self._page_max)
        self._phase_end("metadata_update", start)

    @staticmethod
    def _runs(entries: Sequence[int]) -> list[tuple[int, int]]:
        """Maximal runs of consecutive entries as (first, count)."""
        runs: list[tuple[int, int]] = []
        for e in entries:
            if runs and runs[-1][0] + runs[-1][1] == e:
                runs[-1] = (runs[-1][0], runs[-1][1] + 1)
            else:
                runs.append((e, 1))
        return runs

    def _write_prompt(self, entry: int, key_states: torch.Tensor, value_states: torch.Tensor, start: int,
                      end: int) -> None:
        """Prompt K/V into the slab: a copy on the eviction stream for the
        pinned host slab (quest_offload_cache.py:230-274), in-stream for HBM."""
        if self.kv_residency == "hbm":
            self._key_cache[entry, start:end].copy_(key_states[0, 0])
            self._value_cache[entry, start:end].copy_(value_states[0, 0])
            return
        src_k, src_v = key_states.detach(), value_states.detach()
        ready = torch.cuda.Event()
        ready.record(self._stream())
        with torch.cuda.stream(self.eviction_stream):
            self.eviction_stream.wait_event(ready)
            self._key_cache[entry, start:end].copy_(src_k[0, 0], non_blocking=True)
            self._value_cache[entry, start:end].copy_(src_v[0, 0], non_blocking=True)
            done = torch.cuda.Event()
            done.record(self.eviction_stream)
        src_k.record_stream(self.eviction_stream)
        src_v.record_stream(self.eviction_stream)
        self._host_write_done[entry] = done
        if self.metrics_enabled:
            self.metrics["d2h_bytes"] += 2 * (end - start) * self.geometry.head_dim * src_k.element_size()
            self.metrics["d2h_copy_calls"] += 2

    def _wait_host_writes(self, entries: Sequence[int]) -> None:
        """Order this stream after the slab writes of the entries (a device-side
        wait; the host never blocks)."""
        for entry in entries:
            done = self._host_write_done[entry]
            if done is not None:
                self._stream().wait_event(done)
                self._host_write_done[entry] = None

    # -------------------------------------------------------------- selection
    def _budget(self, old_length: int) -> tuple[int, int]:
        """(candidate_pages, k) of quest_offload_cache.py:326-346; budget_pages
        replaces the fraction when given."""
        _, _, eligible = _window(old_length, self.sink_tokens, self.recent_tokens)
        cand = eligible // self.block_size
        if self.budget_pages is not None:
            budget = min(cand, self.budget_pages)
        else:
            budget = min(cand, max(1, math.ceil(self.budget_fraction * eligible / self.block_size)))
        if self._page_min is None:
            raise RuntimeError("prompt metadata is missing")
        cand = min(cand, int(self._page_min.shape[1]))
        return cand, min(budget, cand)

    def _decode_step(self, old_length: int) -> int:
        if self._prompt_length is None:
            raise RuntimeError("prompt length is missing")
        return old_length - self._prompt_length + 1

    @staticmethod
    def _consecutive(entries: Sequence[int]) -> bool:
        return all(b == a + 1 for a, b in zip(entries, entries[1:]))

    def _metadata(self, entries: Sequence[int], pages: int) -> tuple[torch.Tensor, torch.Tensor]:
        assert self._page_min is not None and self._page_max is not None
        if self._consecutive(entries):
            e0 = entries[0]
            return (self._page_min[e0:e0 + len(entries), :pages], self._page_max[e0:e0 + len(entries), :pages])
        idx = torch.tensor(list(entries), device=self.device)
        return self._page_min[idx, :pages], self._page_max[idx, :pages]

    def _quest_pages(self, q: torch.Tensor, entries: Sequence[int], cand: int, k: int) -> torch.Tensor:
        """Per-head top-k pages of the entries: [G, R, k] int32 on the device."""
        pmin, pmax = self._metadata(entries, cand)
        sel = torch.empty((len(entries), self.num_query_heads_per_kv, k), dtype=torch.int32, device=self.device)
        kernels.quest_select(q, pmin, pmax, k, sel_pages=sel)
        return sel

    def prepare_layer_selection(self, *, entries: list[int], queries: list[torch.Tensor]) -> None:
        """Quest score + top-k for every query head of one decoder layer in
        one launch pair; the page ids stay on the device
        (quest_offload_cache.py:299-401)."""
        if not self.layer_batched_selection:
            return
        q = self._check_layer_queries(entries, queries)
        old_length = self._uniform_length(entries)
        cand, k = self._budget(old_length)
        decode_step = self._decode_step(old_length)
        refresh = (any(self._cached_selected_pages[e] is None for e in entries)
                   or (decode_step - 1) % self.selection_interval == 0)
        if not refresh or k == 0:
            return
        start = self._phase_start()
        sel = self._quest_pages(q, entries, cand, k)
        self._phase_end("selector", start)
        for g, entry in enumerate(entries):
            self._cached_selected_pages[entry] = sel[g:g + 1]
            self._layer_prepared_entries.add(entry)
        if self.metrics_enabled:
            self.metrics["selector_batch_calls"] += 1
            self.metrics["selector_refresh_query_heads"] += len(entries) * self.num_query_heads_per_kv
        self._trace_selection(decode_step, entries, sel)

    def _check_layer_queries(self, entries: Sequence[int], queries: Sequence[torch.Tensor]) -> torch.Tensor:
        if len(entries) != len(queries) or not entries:
            raise ValueError("entries and queries must be non-empty and aligned")
        if len(set(entries)) != len(entries):
            raise ValueError("layer entries must be unique")
        shape = (1, self.num_query_heads_per_kv, 1, self.geometry.head_dim)
        if any(tuple(query.shape) != shape for query in queries):
            raise ValueError("unexpected layer Query shape")
        return torch.stack([query[0, :, 0] for query in queries], dim=0).float().contiguous()

    def _uniform_length(self, entries: Sequence[int]) -> int:
        lengths = {self._logical_lengths[e] for e in entries}
        if len(lengths) != 1:
            raise AssertionError("layer KV entries have unequal logical lengths")
        return lengths.pop()

    def _entry_pages(self, entry: int, query: torch.Tensor, old_length: int) -> Optional[torch.Tensor]:
        """This entry's [1, R, k] page ids for the decode step: the layer-
        prepared ones, a fresh selection, or the cached ones between refreshes
        (quest_offload_cache.py:403-511)."""
        cand, k = self._budget(old_length)
        if k == 0:
            self._layer_prepared_entries.discard(entry)
            return None
        decode_step = self._decode_step(old_length)
        cached = self._cached_selected_pages[entry]
        if entry in self._layer_prepared_entries:
            self._layer_prepared_entries.discard(entry)
            if cached is None:
                raise AssertionError("prepared selection cache is missing")
            return cached
        if cached is None or (decode_step - 1) % self.selection_interval == 0:
            start = self._phase_start()
            q = query[0, :, 0].float().unsqueeze(0).contiguous()
            sel = self._quest_pages(q, [entry], cand, k)
            self._phase_end("selector", start)
            self._cached_selected_pages[entry] = sel
            if self.metrics_enabled:
                self.metrics["selector_refresh_query_heads"] += self.num_query_heads_per_kv
            self._trace_selection(decode_step, [entry], sel)
            return sel
        if self.metrics_enabled:
            self.metrics["selector_reuse_query_heads"] += self.num_query_heads_per_kv
        return cached

    def _history_length(self, old_length: int, k: int) -> int:
        sink_end, recent_start, _ = _window(old_length, self.sink_tokens, self.recent_tokens)
        return sink_end + k * self.block_size + (old_length - recent_start)

    # ---------------------------------------------------------------- update
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: Optional[Dict[str, Any]] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        """Prefill: metadata + slab write, returns the inputs.  Decode: each
        query head's sink ++ pages ++ recent ++ decode token as [1, R, Tmax, D]
        views (quest_offload_cache.py:513-665); get_last_query_head_lengths
        gives the valid lengths."""
        if key_states.shape != value_states.shape or key_states.shape[:2] != (1, 1):
            raise ValueError("expected identical head-wise [1, 1, seq, dim] K/V")
        if key_states.shape[-1] != self.geometry.head_dim or key_states.dtype != self.dtype:
            raise ValueError("K/V head_dim or dtype does not match the cache")
        append_length = int(key_states.shape[-2])
        old_length, new_length = self._bookkeeping.advance(layer_idx, append_length)
        self._seen_tokens = self._bookkeeping.seen_tokens
        self._initialized[layer_idx] = True

        if append_length > 1:
            if old_length != 0:
                raise ValueError("chunked/multiple prefill updates are unsupported")
            if self._prompt_length is None:
                self._prompt_length = append_length
            elif self._prompt_length != append_length:
                raise RuntimeError("cache entries received unequal prompt lengths")
            self._build_metadata(layer_idx, key_states)
            self._write_prompt(layer_idx, key_states, value_states, old_length, new_length)
            return key_states, value_states

        query = None if cache_kwargs is None else cache_kwargs.get("query_states")
        R, D = self.num_query_heads_per_kv, self.geometry.head_dim
        if query is None or tuple(query.shape) != (1, R, 1, D):
            raise ValueError("decode requires post-RoPE query_states")
        self._wait_host_writes([layer_idx])
        sel = self._entry_pages(layer_idx, query, old_length)
        k = 0 if sel is None else int(sel.shape[2])
        history = self._history_length(old_length, k)
        total = history + 1
        self._ensure_pack(total)
        start = self._phase_start()
        cur_k = key_states[0, 0].contiguous()
        cur_v = value_states[0, 0].contiguous()
        kernels.gather_heads(self._key_rows, self._value_rows, sel, cur_k, cur_v, self._pack_rows_k,
                             self._pack_rows_v, entry_row0=self.geometry.row(layer_idx, 0), entry_row_step=0,
                             sink=self.sink_tokens, recent=self.recent_tokens, block_size=self.block_size,
                             length=old_length, num_heads=R, dst_strides=(0, 1, R), error_flag=self._gather_error)
        self._phase_end("gather", start)
        self._append([layer_idx], cur_k, cur_v, old_length)
        self._last_query_head_lengths[layer_idx] = (total,) * R
        if self.metrics_enabled:
            self.metrics["cache_update_calls"] += 1
            self.metrics["selected_history_tokens_total"] += history * R
            self.metrics["attention_valid_tokens_total"] += total * R
            self.metrics["gather_bytes"] += 2 * history * R * D * key_states.element_size()
        assert self._gpu_pack_keys is not None and self._gpu_pack_values is not None
        return (self._gpu_pack_keys[:, :total].transpose(1, 2), self._gpu_pack_values[:, :total].transpose(1, 2))

    def _ensure_pack(self, total: int) -> None:
        R, D = self.num_query_heads_per_kv, self.geometry.head_dim
        if self._gpu_pack_keys is None or self._gpu_pack_keys.shape[1] < total:
            rows = max(total, self.max_selected_tokens_per_query_head + 1)
            self._gpu_pack_keys = torch.empty((1, rows, R, D), dtype=self.dtype, device=self.device)
            self._gpu_pack_values = torch.empty_like(self._gpu_pack_keys)
        self._pack_rows_k = self._gpu_pack_keys.view(-1, D)
        self._pack_rows_v = self._gpu_pack_values.view(-1, D)

    def _append(self, entries: Sequence[int], cur_k: torch.Tensor, cur_v: torch.Tensor, position: int,
                written: bool = False) -> None:
        """The decode tokens [G, D] into slab row `position` of their entries
        (the per-step append of quest_offload_cache.py:633-638), written by a
        kernel on this stream -- through the mapped address for a host slab.
        written: the attention launch already stored the rows (fused append);
        only the bookkeeping and the metadata update remain."""
        start = self._phase_start()
        if written:
            pass
        elif self._consecutive(entries):
            kernels.append_kv(cur_k, cur_v, self._key_cache, self._value_cache, first_entry=entries[0],
                              position=position)
        else:
            for g, entry in enumerate(entries):
                kernels.append_kv(cur_k[g:g + 1], cur_v[g:g + 1], self._key_cache, self._value_cache,
                                  first_entry=entry, position=position)
        self._phase_end("new_kv_append", start)
        if self.metrics_enabled:
            self.metrics["new_kv_append_bytes"] += 2 * cur_k.numel() * cur_k.element_size()
        self._update_decode_metadata(entries, position)

    # ------------------------------------------------------ layer-flat ragged
    def _advance_layer(self, entries: Sequence[int], key_states: Sequence[torch.Tensor],
                       value_states: Sequence[torch.Tensor], queries: Sequence[torch.Tensor]) -> int:
        if not (len(entries) == len(key_states) == len(value_states) == len(queries) and entries):
            raise ValueError("layer entries, K/V, and Queries must be aligned")
        if len(set(entries)) != len(entries):
            raise ValueError("layer entries must be unique")
        D = self.geometry.head_dim
        for key, value in zip(key_states, value_states):
            if key.shape != value.shape or tuple(key.shape) != (1, 1, 1, D):
                raise ValueError("layer decode expects [1, 1, 1, dim] K/V")
        old_lengths = []
        for entry in entries:
            old, _ = self._bookkeeping.advance(entry, 1)
            self._initialized[entry] = True
            old_lengths.append(old)
        self._seen_tokens = self._bookkeeping.seen_tokens
        if len(set(old_lengths)) != 1:
            raise AssertionError("layer KV entries have unequal logical lengths")
        return old_lengths[0]

    def _layer_pages(self, entries: Sequence[int], queries: Sequence[torch.Tensor],
                     old_length: int) -> Optional[torch.Tensor]:
        """[G, R, k] page ids of a layer (prepared, fresh or reused)."""
        parts = [self._entry_pages(e, q, old_length) for e, q in zip(entries, queries)]
        if parts[0] is None:
            return None
        return torch.cat(parts, dim=0)

    def update_layer_flat_ragged(
        self,
        *,
        key_states: list[torch.Tensor],
        value_states: list[torch.Tensor],
        queries: list[torch.Tensor],
        entries: list[int],
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, int, tuple[int, ...]]:
        """All G*R per-query-head histories of a layer as one ragged batch:
        (K[sum T, 1, D], V, cu_seqlens_k int32 [G*R+1] on the device,
        max_seqlen_k, lengths) with segment (g, r) = head r's history ++ the
        decode token (quest_offload_cache.py:724-987)."""
        if not self.layer_flat_ragged_execution:
            raise RuntimeError("layer-flat ragged execution is disabled")
        old_length = self._advance_layer(entries, key_states, value_states, queries)
        self._wait_host_writes(entries)
        G, R, D = len(entries), self.num_query_heads_per_kv, self.geometry.head_dim
        if self._layer_flat_group_count is None:
            self._layer_flat_group_count = G
        elif self._layer_flat_group_count != G:
            raise ValueError("layer KV group count changed after initialization")
        sel = self._layer_pages(entries, queries, old_length)
        k = 0 if sel is None else int(sel.shape[2])
        T = self._history_length(old_length, k) + 1
        total = G * R * T
        if self._flat_keys is None or self._flat_keys.shape[0] < total:
            cap = max(total, G * R * (self.max_selected_tokens_per_query_head + 1))
            self._flat_keys = torch.empty((cap, 1, D), dtype=self.dtype, device=self.device)
            self._flat_values = torch.empty_like(self._flat_keys)
        cur_k = torch.cat([k_[0, 0] for k_ in key_states], dim=0).contiguous()
        cur_v = torch.cat([v_[0, 0] for v_ in value_states], dim=0).contiguous()
        start = self._phase_start()
        fk, fv = self._flat_keys.view(-1, D), self._flat_values.view(-1, D)
        if self._consecutive(entries):
            kernels.gather_heads(self._key_rows, self._value_rows, sel, cur_k, cur_v, fk, fv,
                                 entry_row0=self.geometry.row(entries[0], 0),
                                 entry_row_step=self.geometry.max_cache_len, sink=self.sink_tokens,
                                 recent=self.recent_tokens, block_size=self.block_size, length=old_length,
                                 num_heads=R, dst_strides=(R * T, T, 1), error_flag=self._gather_error)
        else:
            for g, entry in enumerate(entries):
                kernels.gather_heads(self._key_rows, self._value_rows, None if sel is None else sel[g:g + 1],
                                     cur_k[g:g + 1], cur_v[g:g + 1], fk[g * R * T:], fv[g * R * T:],
                                     entry_row0=self.geometry.row(entry, 0), entry_row_step=0,
                                     sink=self.sink_tokens, recent=self.recent_tokens, block_size=self.block_size,
                                     length=old_length, num_heads=R, dst_strides=(0, T, 1),
                                     error_flag=self._gather_error)
        self._phase_end("gather", start)
        self._append(entries, cur_k, cur_v, old_length)
        cu = torch.arange(0, G * R + 1, dtype=torch.int32, device=self.device) * T
        lengths = (T,) * (G * R)
        for entry in entries:
            self._last_query_head_lengths[entry] = (T,) * R
        if self.metrics_enabled:
            self.metrics["cache_update_calls"] += 1
            self.metrics["attention_valid_tokens_total"] += total
        return self._flat_keys[:total], self._flat_values[:total], cu, T, lengths

    # ------------------------------------------------------------ fast path
    def resident_pages(self) -> "kernels.ResidentPages":
        """The HBM resident page cache of every entry (allocated on first use):
        slots for the widest union plan the budget allows, a map over every
        page the metadata can hold, and the resident sink and recent windows."""
        if self._resident is None:
            if self._page_min is None:
                raise RuntimeError("prompt metadata is missing")
            G_all, D = self.geometry.num_entries, self.geometry.head_dim
            pages = max(1, int(self._page_min.shape[1]))
            budget = (self.budget_pages if self.budget_pages is not None else
                      max(1, math.ceil(self.max_selected_history_fraction * max(1, (self.geometry.max_cache_len
                                                                                    - self.sink_tokens)
                                                                                   // self.block_size))))
            slots = max(1, min(pages, self.num_query_heads_per_kv * budget))
            self._resident = kernels.ResidentPages(G_all, slots, pages, D, self.dtype, self.device,
                                                   sink=self.sink_tokens, recent=self.recent_tokens)
        return self._resident

    def resident_stats(self) -> Dict[str, int]:
        """Pages served from the HBM resident cache vs. all union pages read
        (cumulative; synchronizes the device)."""
        if self._resident is None:
            return {"resident_hit_pages": 0, "union_pages": 0}
        st = self._resident.stats.sum(dim=0).tolist()
        return {"resident_hit_pages": int(st[0]), "union_pages": int(st[1])}

    def decode_layer(self, *, queries: torch.Tensor, key_states: torch.Tensor, value_states: torch.Tensor,
                     entries: Sequence[int], softmax_scale: Optional[float] = None,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """One decoder layer's sparse decode in three launches and no host
        sync: Quest selection with the GQA union plan, then the split-K
        attention reading sink ++ union pages ++ recent ++ decode token
        straight from the slab (HBM or zero-copy host), with the decode
        token's append to the slab fused into the attention launch.

        queries [G, R, D] in the cache dtype; key_states/value_states [G, D]
        (the decode token of each entry); entries consecutive.  Returns
        [G, R, D]."""
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
        cand, k = self._budget(old_length)
        e0 = entries[0]
        slab_k = self._key_cache[e0:e0 + G]
        slab_v = self._value_cache[e0:e0 + G]
        if R > 8:
            # sub-groups of at most 8 heads, each with its own union plan: a
            # head attends to its own pages either way, so the output equals
            # one plan over all R heads; every sub-group writes the same row
            if out is None:
                out = torch.empty_like(queries)
            for r0, r1 in kernels.head_chunks(R):
                out[:, r0:r1] = self._decode_pages(queries[:, r0:r1].contiguous(), key_states, value_states, e0,
                                                   slab_k, slab_v, old_length, cand, k, softmax_scale, None)
        else:
            out = self._decode_pages(queries, key_states, value_states, e0, slab_k, slab_v, old_length, cand, k,
                                     softmax_scale, out)
        self._update_decode_metadata(entries, old_length)
        for e in entries:
            self._last_query_head_lengths[e] = None
        return out

    def _decode_pages(self, queries: torch.Tensor, key_states: torch.Tensor, value_states: torch.Tensor, e0: int,
                      slab_k: torch.Tensor, slab_v: torch.Tensor, old_length: int, cand: int, k: int,
                      softmax_scale: Optional[float], out: Optional[torch.Tensor]) -> torch.Tensor:
        """Selection plan + page attention of decode_layer for <= 8 heads."""
        G, R, _ = queries.shape
        entries = list(range(e0, e0 + G))
        width = max(1, min(cand, R * k))
        if k > 0 and cand <= 8192 and not self.previous_token_resident_cache:
            # each head's selection as a page bitmap, ranked by the attention
            # (no union plan to build between the two launches)
            bits = torch.empty((G, R, kernels.sel_bits_words(cand)), dtype=torch.int32, device=self.device)
            start = self._phase_start()
            pmin, pmax = self._metadata(entries, cand)
            kernels.quest_select_bits(queries.float().contiguous(), pmin, pmax, k, bits)
            self._phase_end("selector", start)
            start = self._phase_start()
            result = kernels.decode_attention_pages_bits(
                queries.contiguous(), slab_k, slab_v, bits, cand, max_pages=width, sink=self.sink_tokens,
                recent=self.recent_tokens, block_size=self.block_size, length=old_length, append=True,
                cur_k=key_states.contiguous(), cur_v=value_states.contiguous(), softmax_scale=softmax_scale, out=out)
            self._phase_end("attention", start)
            return result
        plan_pages = torch.empty((G, width), dtype=torch.int32, device=self.device)
        plan_masks = torch.empty((G, width), dtype=torch.uint8, device=self.device)
        plan_counts = torch.zeros((G,), dtype=torch.int32, device=self.device)
        start = self._phase_start()
        if k > 0:
            pmin, pmax = self._metadata(entries, cand)
            kernels.quest_select(queries.float().contiguous(), pmin, pmax, k, plan_pages=plan_pages,
                                 plan_masks=plan_masks, plan_counts=plan_counts)
        self._phase_end("selector", start)
        start = self._phase_start()
        if self.previous_token_resident_cache:
            result = kernels.decode_attention_pages_resident(
                queries.contiguous(), slab_k, slab_v, plan_pages, plan_counts, self.resident_pages().view(e0, G),
                length=old_length, plan_masks=plan_masks, max_pages=width if k > 0 else 0, sink=self.sink_tokens,
                recent=self.recent_tokens, block_size=self.block_size, append=True, cur_k=key_states.contiguous(),
                cur_v=value_states.contiguous(), softmax_scale=softmax_scale, out=out)
        else:
            result = kernels.decode_attention_pages(
                queries.contiguous(), slab_k, slab_v, plan_pages, plan_counts, plan_masks=plan_masks,
                max_pages=width if k > 0 else 0, sink=self.sink_tokens, recent=self.recent_tokens,
                block_size=self.block_size, length=old_length, append_position=old_length,
                cur_k=key_states.contiguous(), cur_v=value_states.contiguous(), softmax_scale=softmax_scale,
                out=out)
        self._phase_end("attention", start)
        return result
