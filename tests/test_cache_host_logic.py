"""Host-side logic of the cache layer (runs without a GPU): slab geometry,
strict sequential bookkeeping, the matched-budget helpers against the
reference's vectors, and the constructors' error behaviour."""

from __future__ import annotations

import json
from pathlib import Path

import pytest
import torch

from headinfer.slab_cache import SequentialCacheState, SlabGeometry

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_slab_geometry_offsets():
    geo = SlabGeometry(num_entries=3, batch_size=1, max_cache_len=10, head_dim=4)
    assert geo.elements_per_entry == 40 and geo.total_elements == 240
    assert geo.bounds("key", 0) == (0, 40) and geo.bounds("key", 2) == (80, 120)
    assert geo.bounds("value", 0) == (120, 160) and geo.bounds("value", 2) == (200, 240)
    assert geo.tensor_shape() == (1, 1, 10, 4)
    assert geo.row(2, 7) == 27
    with pytest.raises(ValueError):
        geo.bounds("query", 0)
    with pytest.raises(IndexError):
        geo.bounds("key", 3)
    with pytest.raises(ValueError):
        SlabGeometry(num_entries=0, batch_size=1, max_cache_len=10, head_dim=4)


def test_sequential_state_strict_order_and_capacity():
    st = SequentialCacheState(2, 5)
    assert st.advance(0, 3) == (0, 3) and st.seen_tokens == 3
    with pytest.raises(ValueError):
        st.advance(0, 1)  # entry 1 is next
    assert st.advance(1, 3) == (0, 3) and st.uniform
    assert st.advance(0, 1) == (3, 4) and st.seen_tokens == 4 and not st.uniform
    assert st.preview(1, 2) == (3, 5)
    with pytest.raises(RuntimeError):
        st.preview(1, 3)
    with pytest.raises(ValueError):
        st.preview(1, 0)
    assert st.logical_lengths == [4, 3] and st.expected_next_entry == 1


def test_matched_budget_helpers_match_reference_vectors():
    from headinfer.twilight_offload_cache import matched_budget_counts, matched_budget_counts_tensor

    cases = json.loads((GOLDEN / "matched_budget_counts.json").read_text())
    for c in cases:
        assert matched_budget_counts(c["desired"], c["target"], c["capacities"]) == c["counts"], c
        if "counts_tensor" in c:
            got = matched_budget_counts_tensor(torch.tensor([c["desired"]]), c["target"], c["capacities"][0])
            assert got.tolist()[0] == c["counts_tensor"], c
    batch = [c for c in cases if "counts_tensor" in c and len(c["desired"]) == 3]
    if len(batch) >= 2:
        cap = min(c["capacities"][0] for c in batch)
        rows = [c for c in batch if c["target"] <= cap][:4]
        if rows:
            tgt = rows[0]["target"]
            rows = [c for c in rows if c["target"] == tgt]
            got = matched_budget_counts_tensor(torch.tensor([c["desired"] for c in rows]), tgt, cap)
            assert got.tolist() == [c["counts_tensor"] for c in rows]
    with pytest.raises(ValueError):
        matched_budget_counts([1, 2], 1, [4, 4])
    with pytest.raises(ValueError):
        matched_budget_counts_tensor(torch.tensor([[1, 2]]), 9, 4)


def test_constructors_require_a_rocm_device():
    from headinfer.quest_offload_cache import QuestTopKOffloadedCache
    from headinfer.twilight_offload_cache import TwilightMatchedBudgetOffloadedCache

    if torch.cuda.is_available():
        pytest.skip("a device is present")
    kw = dict(num_cache_entries=2, max_cache_len=32, head_dim=4, num_query_heads_per_kv=3, dtype=torch.bfloat16,
              device="cuda")
    with pytest.raises(ValueError):
        QuestTopKOffloadedCache(**kw)
    with pytest.raises(ValueError):
        TwilightMatchedBudgetOffloadedCache(**kw)
    with pytest.raises(ValueError):
        TwilightMatchedBudgetOffloadedCache(top_p=1.5, **kw)


@pytest.mark.parametrize("sink,recent,ring", [(64, 256, 256), (64, 257, 512), (0, 1, 1), (16, 0, 1), (4, 100, 128)])
def test_resident_window_sizes(sink, recent, ring):
    """The resident windows hold the sink rows and a ring of the smallest
    power of two >= recent rows (the recent window's recent - 1 history rows
    plus the decode row), state zeroed; a view slices every buffer by group."""
    from headinfer.kernels import ResidentPages

    res = ResidentPages(6, 4, 10, 128, torch.bfloat16, torch.device("cpu"), sink=sink, recent=recent)
    assert res.ring == ring and res.sink == sink
    assert tuple(res.win_k.shape) == (6, sink + ring, 128) and res.win_v.shape == res.win_k.shape
    assert res.win_state.dtype == torch.int32 and not res.win_state.any()
    v = res.view(2, 3)
    assert tuple(v.win_k.shape) == (3, sink + ring, 128) and v.win_k.is_contiguous()
    assert v.win_state.data_ptr() == res.win_state[2].data_ptr() and v.ring == ring
    plain = ResidentPages(6, 4, 10, 128, torch.bfloat16, torch.device("cpu"))
    assert plain.win_k is None and plain.view(0, 2).win_state is None
