"""Side-stream DMA of selected slab rows: the post-selection pipeline of the
reference (``_consume_post_selection_pipeline``, twilight_offload_cache.py:
2053-2455, with its ``selected_kv_h2d_stream``, :417-426).

The zero-copy path reads the selected rows of a pinned host slab from inside
the attention kernels.  This is the other way to bring them over the host
link: the selection comes to the host once, then chunk by chunk the CPU
copies the chunk's rows out of the pinned slab into a pinned staging buffer
(``tw_host_gather_kv``: OpenMP workers, runs of consecutive rows as one
``memcpy``) and a DMA copy on a dedicated stream moves the staging buffer to
HBM.  Two staging buffers alternate, so the CPU gather of chunk c + 1 runs
while the DMA engine copies chunk c and the GPU consumes chunk c - 1: each
chunk's consumer (e.g. the attention of its KV groups) is enqueued on the
compute stream behind that chunk's copy event.  The side stream has the
default priority.
"""

from __future__ import annotations

from typing import Callable, Optional, Sequence

import numpy as np
import torch

from . import kernels

__all__ = ["HostGatherPipeline", "union_rows"]


def union_rows(pages: np.ndarray, *, length: int, sink: int, recent: int, block_size: int) -> np.ndarray:
    """Token positions of a union plan, ascending: [0, sink_end) ++ every page
    p's rows sink + p*bs + [0, bs) ++ [recent_start, length), the window of
    quest_offload_cache.py:330-332 and the page expansion of :484-489."""
    sink_end = min(sink, length)
    recent_start = max(sink_end, length - max(0, recent - 1))
    pg = np.asarray(pages, dtype=np.int64)
    body = (sink + pg[:, None] * block_size + np.arange(block_size, dtype=np.int64)).reshape(-1)
    return np.concatenate([np.arange(sink_end, dtype=np.int64), body,
                           np.arange(recent_start, length, dtype=np.int64)])


class HostGatherPipeline:
    """Chunked host gather + H2D of slab rows on a side stream.

    src_k / src_v: the slab's K and V planes as [rows, D] pinned host tensors
    (row = entry * max_cache_len + position).  ``run`` takes one (rows,
    dst_k, dst_v) triple per chunk -- int64 host row ids and the device
    destinations [n, D] -- and returns after every chunk's copy is enqueued;
    the compute stream then waits on the last copy.  ``on_chunk(c)`` (optional)
    is called right after chunk c's copy is enqueued, with the compute stream
    already waiting on that copy, so work it launches overlaps the later
    chunks' gathers and copies."""

    def __init__(self, device: torch.device, head_dim: int, dtype: torch.dtype, max_rows: int,
                 threads: Optional[int] = None) -> None:
        self.device = torch.device(device)
        self.stream = torch.cuda.Stream(device=self.device)
        self.max_rows = int(max_rows)
        self.threads = threads
        self.stage_k = [torch.empty((self.max_rows, head_dim), dtype=dtype, pin_memory=True) for _ in range(2)]
        self.stage_v = [torch.empty_like(t) for t in self.stage_k]
        self._copied: list[Optional[torch.cuda.Event]] = [None, None]
        self.rows_moved = 0

    def run(self, src_k: torch.Tensor, src_v: torch.Tensor,
            chunks: Sequence[tuple[np.ndarray, torch.Tensor, torch.Tensor]],
            on_chunk: Optional[Callable[[int], None]] = None) -> None:
        if src_k.is_cuda or src_v.is_cuda or not (src_k.is_pinned() and src_v.is_pinned()):
            raise ValueError("the pipeline gathers from a pinned host slab")
        compute = torch.cuda.current_stream(self.device)
        # the side stream must not copy into buffers the compute stream is still writing or reading
        self.stream.wait_stream(compute)
        for c, (rows, dst_k, dst_v) in enumerate(chunks):
            n = int(rows.shape[0])
            if n > self.max_rows:
                raise ValueError(f"chunk of {n} rows exceeds the staging capacity {self.max_rows}")
            if dst_k.shape[0] != n or dst_v.shape[0] != n or not dst_k.is_cuda:
                raise ValueError("each chunk needs device destinations of its row count")
            slot = c % 2
            if self._copied[slot] is not None:
                self._copied[slot].synchronize()  # the DMA that read this staging buffer is done
            if n:
                rows_t = torch.from_numpy(np.ascontiguousarray(rows, dtype=np.int64))
                kernels.host_gather_kv(src_k, src_v, rows_t, self.stage_k[slot][:n], self.stage_v[slot][:n],
                                       threads=self.threads)
                with torch.cuda.stream(self.stream):
                    dst_k.copy_(self.stage_k[slot][:n], non_blocking=True)
                    dst_v.copy_(self.stage_v[slot][:n], non_blocking=True)
                # the destinations belong to the compute stream's allocations
                dst_k.record_stream(self.stream)
                dst_v.record_stream(self.stream)
            ev = torch.cuda.Event()
            ev.record(self.stream)
            self._copied[slot] = ev
            self.rows_moved += n
            if on_chunk is not None:
                compute.wait_event(ev)
                on_chunk(c)
        compute.wait_stream(self.stream)
