"""Slab layout and strict sequential bookkeeping of the offload caches.

Reference: SlabGeometry and SequentialCacheState (slab_cache.py:36-119).
The cache stores every KV head of every layer as one "entry"; entry
e = layer * num_kv_heads + kv_head.  All K rows come first, then all V rows:
one flat tensor of 2 * num_entries * batch * max_cache_len * head_dim
elements, so token t of entry e is row e * max_cache_len + t of its plane.
That row arithmetic is what the gather kernels take (entry_row0 + pos).

Both classes are pure bookkeeping (no device work) and run on the CPU.
"""

from __future__ import annotations

from dataclasses import dataclass, field

__all__ = ["SlabGeometry", "SequentialCacheState"]


@dataclass(frozen=True)
class SlabGeometry:
    """Element offsets of the [2, entries, batch, max_cache_len, head_dim] slab."""

    num_entries: int
    batch_size: int
    max_cache_len: int
    head_dim: int

    def __post_init__(self) -> None:
        for name in ("num_entries", "batch_size", "max_cache_len", "head_dim"):
            value = getattr(self, name)
            if value <= 0:
                raise ValueError(f"{name} must be positive, got {value}")

    @property
    def elements_per_entry(self) -> int:
        return self.batch_size * self.max_cache_len * self.head_dim

    @property
    def total_elements(self) -> int:
        return 2 * self.num_entries * self.elements_per_entry

    def bounds(self, kind: str, entry_idx: int) -> tuple[int, int]:
        """[start, end) element range of one entry's K or V plane."""
        if kind not in ("key", "value"):
            raise ValueError(f"kind must be 'key' or 'value', got {kind!r}")
        if not 0 <= entry_idx < self.num_entries:
            raise IndexError(f"entry_idx {entry_idx} outside [0, {self.num_entries})")
        plane = 0 if kind == "key" else 1
        start = (plane * self.num_entries + entry_idx) * self.elements_per_entry
        return start, start + self.elements_per_entry

    def tensor_shape(self) -> tuple[int, int, int, int]:
        """Shape of one entry's K or V view: [batch, 1, max_cache_len, head_dim]."""
        return (self.batch_size, 1, self.max_cache_len, self.head_dim)

    def row(self, entry_idx: int, position: int) -> int:
        """Row of (entry, position) within a plane viewed as [rows, head_dim]."""
        return entry_idx * self.batch_size * self.max_cache_len + position


@dataclass
class SequentialCacheState:
    """Logical lengths under the strict round-robin entry order.

    Entries are updated 0, 1, ..., num_entries - 1, 0, 1, ...; any other order
    raises ValueError, appending past the capacity raises RuntimeError.
    seen_tokens counts the tokens appended to entry 0."""

    num_entries: int
    allocated_capacity: int
    logical_lengths: list[int] = field(init=False)
    expected_next_entry: int = field(init=False, default=0)
    write_position: int = field(init=False, default=0)
    seen_tokens: int = field(init=False, default=0)

    def __post_init__(self) -> None:
        if self.num_entries <= 0 or self.allocated_capacity <= 0:
            raise ValueError("num_entries and allocated_capacity must be positive")
        self.logical_lengths = [0] * self.num_entries

    def preview(self, entry_idx: int, append_length: int) -> tuple[int, int]:
        """(old_length, new_length) of an append, validated but not applied."""
        if entry_idx != self.expected_next_entry:
            raise ValueError("strict sequential head-wise update violated: "
                             f"expected {self.expected_next_entry}, got {entry_idx}")
        if append_length <= 0:
            raise ValueError("append_length must be positive")
        old = self.logical_lengths[entry_idx]
        new = old + append_length
        if new > self.allocated_capacity:
            raise RuntimeError(f"cache capacity exceeded: {old} + {append_length} > {self.allocated_capacity}")
        return old, new

    def advance(self, entry_idx: int, append_length: int) -> tuple[int, int]:
        old, new = self.preview(entry_idx, append_length)
        self.write_position = old
        self.logical_lengths[entry_idx] = new
        if entry_idx == 0:
            self.seen_tokens += append_length
        self.expected_next_entry = (entry_idx + 1) % self.num_entries
        return old, new

    @property
    def uniform(self) -> bool:
        return len(set(self.logical_lengths)) == 1
