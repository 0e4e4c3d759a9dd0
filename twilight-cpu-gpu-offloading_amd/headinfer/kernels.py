"""Tensor-level wrappers of the gfx950 kernels (the C ABI in
include/twilight_hip.h).

Every wrapper validates shapes, dtypes, devices and contiguity the way the
reference's Triton wrappers do (e.g. twilight_fused_quest.py:35-46,
twilight_fused_qk.py:80-101), enqueues on torch's current stream and never
synchronizes.  There is no CPU path: tensors must live on a ROCm device (or,
for the zero-copy host path, in pinned host memory).
"""

from __future__ import annotations

import functools
import math
from typing import Optional

import torch

from . import _native
from ._native import check, hip, on_device, ptr, stream_handle

_KEY_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _dt(t: torch.Tensor) -> int:
    try:
        return _native.DTYPE_CODES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}") from None


def _require_device(*tensors: Optional[torch.Tensor], what: str) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"{what} requires ROCm device tensors (got {t.device})")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"{what} requires tensors on one device")
    if device is None:
        raise ValueError(f"{what}: no device tensor given")
    return device


def _require_contiguous(*tensors: Optional[torch.Tensor], what: str) -> None:
    for t in tensors:
        if t is not None and not t.is_contiguous():
            raise ValueError(f"{what} requires contiguous tensors")


class _Workspace:
    """Per-device, per-purpose scratch buffers.  Allocated zeroed once; the
    kernels return their arrival counters to zero after every launch.

    A buffer that a larger request outgrows is kept, never freed: a captured
    HIP graph holds its raw address, and replaying that graph after the
    replacement must still write into memory nobody else owns (with counters
    still at zero).  Sizes double, so the retired buffers together are
    smaller than the live one."""

    def __init__(self) -> None:
        self._buffers: dict[tuple, torch.Tensor] = {}
        self._retired: list[torch.Tensor] = []

    def get(self, device: torch.device, name: str, nbytes: int) -> torch.Tensor:
        key = (device, name)
        buf = self._buffers.get(key)
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 1 << 16)
            if buf is not None:
                size = max(size, 2 * buf.numel())
                self._retired.append(buf)
            buf = torch.zeros(size, dtype=torch.uint8, device=device)
            self._buffers[key] = buf
        return buf


WORKSPACE = _Workspace()


def head_chunks(R: int, width: int = 8) -> list[tuple[int, int]]:
    """[r0, r1) ranges splitting R query heads into ceil(R / width) nearly
    equal sub-groups of at most `width` heads (the kernels' per-group limit)."""
    n = -(-R // width)
    return [(R * i // n, R * (i + 1) // n) for i in range(n)]


# --------------------------------------------------------------- metadata
def build_page_metadata(
    keys: torch.Tensor,
    *,
    sink: int,
    block_size: int,
    page_min: Optional[torch.Tensor] = None,
    page_max: Optional[torch.Tensor] = None,
    packed: Optional[torch.Tensor] = None,
    scale: Optional[torch.Tensor] = None,
    minimum: Optional[torch.Tensor] = None,
) -> None:
    """Prompt metadata of n entries in one launch (page min/max and INT4 keys).

    keys: [E, T, D] (or [T, D]); page_min/page_max: [E, >=P, D];
    packed: [E, >=T, D/2] uint8; scale/minimum: [E, >=T].  Any of the two
    output groups may be omitted."""
    if keys.ndim == 2:
        keys = keys.unsqueeze(0)
    if keys.ndim != 3 or keys.dtype not in _KEY_DTYPES:
        raise ValueError("keys must be [entries, tokens, dim] fp16/bf16/fp32")
    E, T, D = keys.shape
    if D % 2:
        raise ValueError("head_dim must be even")
    if keys.stride(2) != 1 or keys.stride(1) != D:
        raise ValueError("keys rows must be contiguous")
    dev = _require_device(keys, page_min, page_max, packed, scale, minimum, what="build_page_metadata")
    pages = (T - sink) // block_size if T > sink else 0
    pe = 0
    if page_min is not None:
        if page_max is None or page_min.shape != page_max.shape or page_min.dtype != keys.dtype:
            raise ValueError("page_min/page_max must match each other and the key dtype")
        if page_min.ndim == 2:
            page_min, page_max = page_min.unsqueeze(0), page_max.unsqueeze(0)
        if page_min.shape[0] != E or page_min.shape[1] < pages or page_min.shape[2] != D:
            raise ValueError("page metadata buffers are too small")
        if page_min.stride(2) != 1 or page_min.stride(1) != D or page_max.stride() != page_min.stride():
            raise ValueError("page metadata buffers must be row-contiguous")
        pe = page_min.stride(0)
    qe = 0
    if packed is not None:
        if scale is None or minimum is None or scale.dtype != keys.dtype or minimum.dtype != keys.dtype:
            raise ValueError("INT4 outputs must be given together in the key dtype")
        if packed.ndim == 2:
            packed, scale, minimum = packed.unsqueeze(0), scale.unsqueeze(0), minimum.unsqueeze(0)
        if packed.dtype != torch.uint8 or packed.shape[0] != E or packed.shape[1] < T or packed.shape[2] != D // 2:
            raise ValueError("packed buffer has the wrong shape")
        if packed.stride(2) != 1 or packed.stride(1) != D // 2:
            raise ValueError("packed rows must be contiguous")
        if packed.stride(0) % (D // 2):
            raise ValueError("packed entry stride must be a whole number of rows")
        qe = packed.stride(0) // (D // 2)
        if scale.stride(-1) != 1 or minimum.stride(-1) != 1 or scale.stride(0) != qe or minimum.stride(0) != qe:
            raise ValueError("scale/minimum must share the packed entry stride")
    elif scale is not None or minimum is not None:
        raise ValueError("INT4 outputs must be given together")
    if page_min is None and packed is None:
        return
    with on_device(dev):
        check(hip().tw_build_page_metadata(ptr(keys), keys.stride(0), E, T, D, _dt(keys), sink, block_size,
                                           ptr(page_min), ptr(page_max), pe, ptr(packed), ptr(scale), ptr(minimum),
                                           qe, stream_handle(dev)), "build_page_metadata")


def update_page_metadata(
    keys: torch.Tensor,
    *,
    first_entry: int,
    n_entries: int,
    position: int,
    sink: int,
    block_size: int,
    page_min: Optional[torch.Tensor] = None,
    page_max: Optional[torch.Tensor] = None,
    packed: Optional[torch.Tensor] = None,
    scale: Optional[torch.Tensor] = None,
    minimum: Optional[torch.Tensor] = None,
    device: Optional[torch.device] = None,
) -> None:
    """Decode-time metadata of entries [first_entry, first_entry + n_entries)
    after row `position` was written: that row's INT4 code and, when the row
    completes a page, the page's min/max (equal to a rebuild over
    position + 1 rows).  keys: the K plane [E, Lmax, D] (HBM or pinned
    host); page_min/page_max [E, P, D]; packed [E, T, D/2] with scale/minimum
    [E, T], indexed by entry like keys."""
    if keys.ndim != 3 or keys.dtype not in _KEY_DTYPES or keys.stride(2) != 1 or keys.stride(1) != keys.shape[2]:
        raise ValueError("keys must be a row-contiguous [E, Lmax, D] plane")
    E, Lmax, D = keys.shape
    if n_entries <= 0 or first_entry < 0 or first_entry + n_entries > E or not 0 <= position < Lmax:
        raise ValueError("update target outside the cache")
    pe = qe = 0
    pmin_p = pmax_p = pk_p = sc_p = mn_p = None
    e0 = first_entry
    if page_min is not None:
        if page_max is None or page_min.shape != page_max.shape or page_min.dtype != keys.dtype \
                or page_min.ndim != 3 or page_min.shape[0] != E or page_min.shape[2] != D \
                or page_min.stride(2) != 1 or page_min.stride(1) != D or page_max.stride() != page_min.stride():
            raise ValueError("page_min/page_max must be row-contiguous [E, P, D] in the key dtype")
        completes = position >= sink and (position - sink + 1) % block_size == 0
        if completes and (position - sink) // block_size >= page_min.shape[1]:
            raise ValueError("page metadata buffers are too small")
        pe = page_min.stride(0)
        pmin_p, pmax_p = ptr(page_min[e0]), ptr(page_max[e0])
    elif page_max is not None:
        raise ValueError("page_min/page_max go together")
    if packed is not None:
        if scale is None or minimum is None or scale.dtype != keys.dtype or minimum.dtype != keys.dtype:
            raise ValueError("INT4 outputs must be given together in the key dtype")
        if packed.dtype != torch.uint8 or packed.ndim != 3 or packed.shape[0] != E or packed.shape[2] != D // 2 \
                or packed.shape[1] <= position or packed.stride(2) != 1 or packed.stride(1) != D // 2 \
                or packed.stride(0) % (D // 2):
            raise ValueError("packed must be row-contiguous [E, > position, D/2] uint8")
        qe = packed.stride(0) // (D // 2)
        if scale.stride(-1) != 1 or minimum.stride(-1) != 1 or scale.stride(0) != qe or minimum.stride(0) != qe:
            raise ValueError("scale/minimum must share the packed entry stride")
        pk_p, sc_p, mn_p = ptr(packed[e0]), ptr(scale[e0]), ptr(minimum[e0])
    elif scale is not None or minimum is not None:
        raise ValueError("INT4 outputs must be given together")
    if pmin_p is None and pk_p is None:
        return
    dev = _require_device(page_min, page_max, packed, scale, minimum, what="update_page_metadata")
    kp = ptr(keys) if keys.is_cuda else host_device_pointer(keys)
    kp += e0 * keys.stride(0) * keys.element_size()
    with on_device(dev):
        check(hip().tw_update_page_metadata(kp, keys.stride(0), n_entries, position, D, _dt(keys), sink,
                                            block_size, pmin_p, pmax_p, pe, pk_p, sc_p, mn_p, qe,
                                            stream_handle(dev)), "update_page_metadata")


def update_page_metadata_ragged(
    keys: torch.Tensor,
    positions: torch.Tensor,
    *,
    first_entry: int,
    sink: int,
    block_size: int,
    page_min: Optional[torch.Tensor] = None,
    page_max: Optional[torch.Tensor] = None,
    packed: Optional[torch.Tensor] = None,
    scale: Optional[torch.Tensor] = None,
    minimum: Optional[torch.Tensor] = None,
) -> None:
    """update_page_metadata for entries [first_entry, first_entry + n) whose
    new rows are positions [n] (int32, device); rows or pages beyond the
    buffers are skipped."""
    if keys.ndim != 3 or keys.dtype not in _KEY_DTYPES or keys.stride(2) != 1 or keys.stride(1) != keys.shape[2]:
        raise ValueError("keys must be a row-contiguous [E, Lmax, D] plane")
    E, Lmax, D = keys.shape
    if positions.dtype != torch.int32 or positions.ndim != 1 or not positions.is_contiguous():
        raise ValueError("positions must be contiguous [n] int32")
    n = positions.shape[0]
    if n <= 0 or first_entry < 0 or first_entry + n > E:
        raise ValueError("update target outside the cache")
    e0 = first_entry
    max_position = Lmax - 1
    pmin_p = pmax_p = pk_p = sc_p = mn_p = None
    pe = qe = max_pages = 0
    if page_min is not None:
        if page_max is None or page_min.shape != page_max.shape or page_min.dtype != keys.dtype \
                or page_min.ndim != 3 or page_min.shape[0] != E or page_min.shape[2] != D \
                or page_min.stride(2) != 1 or page_min.stride(1) != D or page_max.stride() != page_min.stride():
            raise ValueError("page_min/page_max must be row-contiguous [E, P, D] in the key dtype")
        pe, max_pages = page_min.stride(0), page_min.shape[1]
        pmin_p, pmax_p = ptr(page_min[e0]), ptr(page_max[e0])
    elif page_max is not None:
        raise ValueError("page_min/page_max go together")
    if packed is not None:
        if scale is None or minimum is None or scale.dtype != keys.dtype or minimum.dtype != keys.dtype:
            raise ValueError("INT4 outputs must be given together in the key dtype")
        if packed.dtype != torch.uint8 or packed.ndim != 3 or packed.shape[0] != E or packed.shape[2] != D // 2 \
                or packed.stride(2) != 1 or packed.stride(1) != D // 2 or packed.stride(0) % (D // 2):
            raise ValueError("packed must be row-contiguous [E, T, D/2] uint8")
        qe = packed.stride(0) // (D // 2)
        if scale.stride(-1) != 1 or minimum.stride(-1) != 1 or scale.stride(0) != qe or minimum.stride(0) != qe:
            raise ValueError("scale/minimum must share the packed entry stride")
        max_position = min(max_position, packed.shape[1] - 1)
        pk_p, sc_p, mn_p = ptr(packed[e0]), ptr(scale[e0]), ptr(minimum[e0])
    elif scale is not None or minimum is not None:
        raise ValueError("INT4 outputs must be given together")
    if pmin_p is None and pk_p is None:
        return
    dev = _require_device(positions, page_min, page_max, packed, scale, minimum, what="update_page_metadata_ragged")
    kp = ptr(keys) if keys.is_cuda else host_device_pointer(keys)
    kp += e0 * keys.stride(0) * keys.element_size()
    with on_device(dev):
        check(hip().tw_update_page_metadata_ragged(kp, keys.stride(0), n, ptr(positions), max_position, D,
                                                   _dt(keys), sink, block_size, pmin_p, pmax_p, max_pages, pe, pk_p,
                                                   sc_p, mn_p, qe, stream_handle(dev)), "update_page_metadata_ragged")


def affine_int4_pack(keys: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per-token affine INT4 (twilight_offload_cache.py:25-37) on the GPU."""
    if keys.ndim != 2 or keys.shape[-1] % 2:
        raise ValueError("keys must be [tokens, even head_dim]")
    T, D = keys.shape
    keys = keys.contiguous()
    packed = torch.empty((T, D // 2), dtype=torch.uint8, device=keys.device)
    scale = torch.empty((T,), dtype=keys.dtype, device=keys.device)
    minimum = torch.empty((T,), dtype=keys.dtype, device=keys.device)
    build_page_metadata(keys, sink=T, block_size=1, packed=packed, scale=scale, minimum=minimum)
    return packed, scale, minimum


def affine_int4_dequantize(packed: torch.Tensor, scale: torch.Tensor, minimum: torch.Tensor) -> torch.Tensor:
    """twilight_offload_cache.py:40-47 on the GPU; returns fp32 [..., D]."""
    if packed.dtype != torch.uint8 or scale.shape != packed.shape[:-1] or minimum.shape != scale.shape:
        raise ValueError("incompatible packed/scale/minimum")
    if scale.dtype != minimum.dtype:
        raise ValueError("scale and minimum dtypes differ")
    dev = _require_device(packed, scale, minimum, what="affine_int4_dequantize")
    packed, scale, minimum = packed.contiguous(), scale.contiguous(), minimum.contiguous()
    D = packed.shape[-1] * 2
    N = scale.numel()
    out = torch.empty((*packed.shape[:-1], D), dtype=torch.float32, device=dev)
    with on_device(dev):
        check(hip().tw_int4_dequantize(ptr(packed), ptr(scale), ptr(minimum), _dt(scale), N, D, ptr(out),
                                       stream_handle(dev)), "affine_int4_dequantize")
    return out


# ------------------------------------------------------------------ Quest
def _check_score_inputs(q, page_min, page_max, what):
    if q.ndim != 3 or q.dtype != torch.float32:
        raise ValueError(f"{what}: q must be [G, R, D] fp32")
    if page_min.dtype not in _KEY_DTYPES or page_max.dtype != page_min.dtype:
        raise ValueError(f"{what}: unsupported metadata dtypes")
    if page_min.ndim != 3 or page_min.shape != page_max.shape or page_min.shape[0] != q.shape[0] \
            or page_min.shape[2] != q.shape[2]:
        raise ValueError(f"{what}: metadata must be [G, P, D] matching q")
    if page_min.stride(2) != 1 or page_min.stride(1) != q.shape[2] or page_max.stride() != page_min.stride():
        raise ValueError(f"{what}: metadata rows must be contiguous")
    if not q.is_contiguous():
        raise ValueError(f"{what}: q must be contiguous")
    if q.shape[2] % 2 or q.shape[2] > 256:
        raise ValueError(f"{what}: head_dim must be even and <= 256")


def fused_quest_score(q: torch.Tensor, page_min: torch.Tensor, page_max: torch.Tensor, *,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Quest upper-bound page score in the reference's explicit order
    (twilight_fused_quest.py:35-46).  q [G,R,D] fp32, lo/hi [G,P,D]; out
    (optional) a contiguous [G,R,P] fp32 tensor to write."""
    _check_score_inputs(q, page_min, page_max, "fused_quest_score")
    dev = _require_device(q, page_min, page_max, out, what="fused_quest_score")
    G, R, D = q.shape
    P = page_min.shape[1]
    if out is None:
        out = torch.empty((G, R, P), dtype=torch.float32, device=dev)
    elif out.dtype != torch.float32 or tuple(out.shape) != (G, R, P) or not out.is_contiguous():
        raise ValueError("fused_quest_score out must be a contiguous [G, R, P] float32 tensor")
    if P == 0:
        return out
    with on_device(dev):
        check(hip().tw_quest_score(ptr(q), ptr(page_min), ptr(page_max), _dt(page_min), G, R, P, D,
                                   page_min.stride(0), ptr(out), stream_handle(dev)), "fused_quest_score")
    return out


def topk_sorted(scores: torch.Tensor, k: int) -> torch.Tensor:
    """torch.topk(scores, k, sorted=False).indices.sort().values with ties to
    the lowest index (quest_offload_cache.py:373-374).  int64 [..., k]."""
    if scores.dtype != torch.float32:
        raise ValueError("scores must be fp32")
    dev = _require_device(scores, what="topk_sorted")
    P = scores.shape[-1]
    if not 1 <= k <= P:
        raise ValueError("k must be in [1, P]")
    flat = scores.reshape(-1, P)
    if flat.stride(1) != 1:
        flat = flat.contiguous()
    out = torch.empty((flat.shape[0], k), dtype=torch.int64, device=dev)
    nbytes = hip().tw_topk_sorted_workspace_size(flat.shape[0], P)
    ws = WORKSPACE.get(dev, "topk_sorted", nbytes) if nbytes else None
    with on_device(dev):
        check(hip().tw_topk_sorted(ptr(flat), flat.shape[0], P, flat.stride(0), k, ptr(out), ptr(ws),
                                   0 if ws is None else ws.numel(), stream_handle(dev)), "topk_sorted")
    return out.view(*scores.shape[:-1], k)


def quest_select(
    q: torch.Tensor,
    page_min: torch.Tensor,
    page_max: torch.Tensor,
    k: int,
    *,
    scores: Optional[torch.Tensor] = None,
    sel_pages: Optional[torch.Tensor] = None,
    plan_pages: Optional[torch.Tensor] = None,
    plan_masks: Optional[torch.Tensor] = None,
    plan_counts: Optional[torch.Tensor] = None,
    rows: Optional[torch.Tensor] = None,
    row_masks: Optional[torch.Tensor] = None,
    row_counts: Optional[torch.Tensor] = None,
    sink: int = 0,
    recent: int = 1,
    block_size: int = 1,
    length: int = 0,
    append_position: int = -1,
) -> None:
    """Quest score + top-k + GQA union plan for one layer (two launches).

    page_min/page_max: [G, P, D] views (P pages are scored).  Outputs are
    caller-allocated: scores [G,R,P] fp32, sel_pages [G,R,k] int32, the union
    plan plan_pages/plan_masks [G, >=min(P, R*k)] int32/uint8 with
    plan_counts [G] int32, the row plan rows/row_masks [G, stride]
    int32/uint8 with row_counts [G] int32."""
    _check_score_inputs(q, page_min, page_max, "quest_select")
    dev = _require_device(q, page_min, page_max, scores, sel_pages, plan_pages, plan_masks, plan_counts, rows,
                          row_masks, row_counts, what="quest_select")
    G, R, D = q.shape
    P = page_min.shape[1]
    if not 1 <= k <= P:
        raise ValueError("k must be in [1, P]")
    for t, dt, shape in ((scores, torch.float32, (G, R, P)), (sel_pages, torch.int32, (G, R, k)),
                         (row_counts, torch.int32, (G,)), (plan_counts, torch.int32, (G,))):
        if t is not None and (t.dtype != dt or tuple(t.shape) != shape or not t.is_contiguous()):
            raise ValueError("quest_select output has the wrong dtype/shape")
    stride = 0
    if rows is not None:
        if rows.dtype != torch.int32 or rows.ndim != 2 or rows.shape[0] != G or rows.stride(1) != 1:
            raise ValueError("rows must be [G, stride] int32")
        stride = rows.stride(0)
        if row_masks is not None and (row_masks.dtype != torch.uint8 or row_masks.shape != rows.shape
                                      or row_masks.stride() != rows.stride()):
            raise ValueError("row_masks must match rows")
    plan_stride = 0
    if plan_pages is not None:
        if plan_pages.dtype != torch.int32 or plan_pages.ndim != 2 or plan_pages.shape[0] != G \
                or plan_pages.stride(1) != 1:
            raise ValueError("plan_pages must be [G, stride] int32")
        plan_stride = plan_pages.stride(0)
        if plan_masks is not None and (plan_masks.dtype != torch.uint8 or plan_masks.shape != plan_pages.shape
                                       or plan_masks.stride() != plan_pages.stride()):
            raise ValueError("plan_masks must match plan_pages")
    nbytes = hip().tw_quest_select_workspace_size(G, R, P)
    ws = WORKSPACE.get(dev, "quest_select", nbytes)
    with on_device(dev):
        check(hip().tw_quest_select(ptr(q), ptr(page_min), ptr(page_max), _dt(page_min), G, R, P, D,
                                    page_min.stride(0), k, ptr(scores), ptr(sel_pages), ptr(plan_pages),
                                    ptr(plan_masks), ptr(plan_counts), plan_stride, ptr(rows), ptr(row_masks),
                                    ptr(row_counts), stride, sink, recent, block_size, length, append_position,
                                    ptr(ws), ws.numel(), stream_handle(dev)), "quest_select")


def quest_select_ragged(
    q: torch.Tensor,
    page_min: torch.Tensor,
    page_max: torch.Tensor,
    lengths: torch.Tensor,
    k: int,
    *,
    sink: int,
    recent: int,
    block_size: int,
    sel_pages: Optional[torch.Tensor] = None,
    plan_pages: Optional[torch.Tensor] = None,
    plan_masks: Optional[torch.Tensor] = None,
    plan_counts: Optional[torch.Tensor] = None,
) -> None:
    """quest_select over G groups of different lengths (lengths [G] int32 on
    the device): group g scores its own candidate pages (at most the P of
    page_min [G, P, D]) and keeps min(k, its pages) per head; sel_pages slots
    beyond that are -1.  Union plan as in quest_select."""
    _check_score_inputs(q, page_min, page_max, "quest_select_ragged")
    dev = _require_device(q, page_min, page_max, lengths, sel_pages, plan_pages, plan_masks, plan_counts,
                          what="quest_select_ragged")
    G, R, D = q.shape
    P = page_min.shape[1]
    if not 1 <= k <= P:
        raise ValueError("k must be in [1, P]")
    if lengths.dtype != torch.int32 or tuple(lengths.shape) != (G,) or not lengths.is_contiguous():
        raise ValueError("lengths must be contiguous [G] int32")
    for t, dt, shape in ((sel_pages, torch.int32, (G, R, k)), (plan_counts, torch.int32, (G,))):
        if t is not None and (t.dtype != dt or tuple(t.shape) != shape or not t.is_contiguous()):
            raise ValueError("quest_select_ragged output has the wrong dtype/shape")
    plan_stride = 0
    if plan_pages is not None:
        if plan_pages.dtype != torch.int32 or plan_pages.ndim != 2 or plan_pages.shape[0] != G \
                or plan_pages.stride(1) != 1:
            raise ValueError("plan_pages must be [G, stride] int32")
        plan_stride = plan_pages.stride(0)
        if plan_masks is not None and (plan_masks.dtype != torch.uint8 or plan_masks.shape != plan_pages.shape
                                       or plan_masks.stride() != plan_pages.stride()):
            raise ValueError("plan_masks must match plan_pages")
    nbytes = hip().tw_quest_select_workspace_size(G, R, P)
    ws = WORKSPACE.get(dev, "quest_select", nbytes)
    with on_device(dev):
        check(hip().tw_quest_select_ragged(ptr(q), ptr(page_min), ptr(page_max), _dt(page_min), G, R, P, D,
                                           page_min.stride(0), ptr(lengths), k, ptr(sel_pages), ptr(plan_pages),
                                           ptr(plan_masks), ptr(plan_counts), plan_stride, sink, recent, block_size,
                                           ptr(ws), ws.numel(), stream_handle(dev)), "quest_select_ragged")


def sel_bits_words(P: int) -> int:
    """32-bit words of one selection-bitmap row over P pages (whole 64-bit
    words)."""
    return 2 * ((P + 63) // 64)


def quest_select_bits(
    q: torch.Tensor,
    page_min: torch.Tensor,
    page_max: torch.Tensor,
    k: int,
    sel_bits: torch.Tensor,
    *,
    lengths: Optional[torch.Tensor] = None,
    scores: Optional[torch.Tensor] = None,
    sel_pages: Optional[torch.Tensor] = None,
    sink: int = 0,
    recent: int = 1,
    block_size: int = 1,
) -> None:
    """Quest score + top-k with each head's selection written as a page
    bitmap (two launches, no union plan): bit p of sel_bits[g, r] (int32
    words, [G, R, >= sel_bits_words(P)]) is set when head r of group g chose
    page p.  lengths ([G] int32, device, optional) selects per group as
    quest_select_ragged.  P <= 8192."""
    _check_score_inputs(q, page_min, page_max, "quest_select_bits")
    dev = _require_device(q, page_min, page_max, lengths, scores, sel_pages, sel_bits, what="quest_select_bits")
    G, R, D = q.shape
    P = page_min.shape[1]
    if not 1 <= k <= P:
        raise ValueError("k must be in [1, P]")
    if P > 8192:
        raise ValueError("quest_select_bits takes at most 8192 pages (use quest_select)")
    if sel_bits.dtype != torch.int32 or sel_bits.ndim != 3 or tuple(sel_bits.shape[:2]) != (G, R) \
            or sel_bits.shape[2] < sel_bits_words(P) or sel_bits.stride(2) != 1 \
            or sel_bits.stride(0) != R * sel_bits.stride(1) or sel_bits.stride(1) % 2 or sel_bits.data_ptr() % 8:
        raise ValueError("sel_bits must be [G, R, >= sel_bits_words(P)] int32 with 8-byte aligned rows")
    for t, dt, shape in ((scores, torch.float32, (G, R, P)), (sel_pages, torch.int32, (G, R, k))):
        if t is not None and (t.dtype != dt or tuple(t.shape) != shape or not t.is_contiguous()):
            raise ValueError("quest_select_bits output has the wrong dtype/shape")
    if lengths is not None and (lengths.dtype != torch.int32 or tuple(lengths.shape) != (G,)
                                or not lengths.is_contiguous()):
        raise ValueError("lengths must be contiguous [G] int32")
    nbytes = hip().tw_quest_select_workspace_size(G, R, P)
    ws = WORKSPACE.get(dev, "quest_select", nbytes)
    with on_device(dev):
        check(hip().tw_quest_select_bits(ptr(q), ptr(page_min), ptr(page_max), _dt(page_min), G, R, P, D,
                                         page_min.stride(0), ptr(lengths), k, ptr(scores), ptr(sel_pages),
                                         ptr(sel_bits), sel_bits.stride(1), sink, recent, block_size, ptr(ws),
                                         ws.numel(), stream_handle(dev)), "quest_select_bits")


# ---------------------------------------------------------------- Twilight
def twilight_qk(
    q: torch.Tensor,
    packed: torch.Tensor,
    scale: torch.Tensor,
    minimum: torch.Tensor,
    plan_pages: torch.Tensor,
    plan_masks: torch.Tensor,
    plan_counts: torch.Tensor,
    b0_pages: int,
    *,
    sink: int,
    block_size: int,
    qk_scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
    slot_u: Optional[torch.Tensor] = None,
    page_rows: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """INT4 QK estimate of every head over its B0 candidates (one launch).

    q [G,R,D] fp32; packed [G, >=T, D/2] uint8 with scale/minimum [G, >=T]
    (build_page_metadata's INT4 outputs); the stage-1 union plan of
    quest_select with k = b0_pages.  Returns logits [G, R, b0_pages*bs] fp32
    in candidate order (each head's pages ascending, block_size rows each).
    slot_u [G, R, b0_pages] int32 and page_rows [G, plan stride] int32 (both
    or neither): the union index of every head's B0 slot, and cleared row
    masks of the union pages, for twilight_select_pages."""
    if q.ndim != 3 or q.dtype != torch.float32 or not q.is_contiguous():
        raise ValueError("q must be contiguous [G, R, D] fp32")
    G, R, D = q.shape
    if packed.dtype != torch.uint8 or packed.ndim != 3 or packed.shape[0] != G or packed.shape[2] != D // 2:
        raise ValueError("packed must be [G, T, D/2] uint8")
    if packed.stride(2) != 1 or packed.stride(1) != D // 2 or packed.stride(0) % (D // 2):
        raise ValueError("packed rows must be contiguous")
    qe = packed.stride(0) // (D // 2)
    if scale.dtype not in _KEY_DTYPES or minimum.dtype != scale.dtype or scale.ndim != 2:
        raise ValueError("scale/minimum must be [G, T] in one key dtype")
    if scale.stride(1) != 1 or minimum.stride(1) != 1 or scale.stride(0) != qe or minimum.stride(0) != qe:
        raise ValueError("scale/minimum must share the packed entry stride")
    if plan_pages.dtype != torch.int32 or plan_pages.ndim != 2 or plan_pages.shape[0] != G \
            or plan_pages.stride(1) != 1 or plan_masks.stride() != plan_pages.stride() \
            or plan_masks.dtype != torch.uint8 or plan_counts.dtype != torch.int32 or plan_counts.shape != (G,):
        raise ValueError("plan_pages/plan_masks/plan_counts must be quest_select's union plan")
    dev = _require_device(q, packed, scale, minimum, plan_pages, plan_masks, plan_counts, out, what="twilight_qk")
    N = b0_pages * block_size
    if out is None:
        out = torch.empty((G, R, N), dtype=torch.float32, device=dev)
    elif out.dtype != torch.float32 or tuple(out.shape) != (G, R, N) or not out.is_contiguous():
        raise ValueError("out must be contiguous [G, R, b0_pages*block_size] fp32")
    qs = _default_qk_scale(D) if qk_scale is None else float(qk_scale)
    if (slot_u is None) != (page_rows is None):
        raise ValueError("slot_u and page_rows go together")
    if slot_u is not None:
        if slot_u.dtype != torch.int32 or tuple(slot_u.shape) != (G, R, b0_pages) or not slot_u.is_contiguous():
            raise ValueError("slot_u must be contiguous [G, R, b0_pages] int32")
        if page_rows.dtype != torch.int32 or tuple(page_rows.shape) != tuple(plan_pages.shape) \
                or page_rows.stride() != plan_pages.stride():
            raise ValueError("page_rows must be int32 shaped and strided like plan_pages")
        _require_device(slot_u, page_rows, what="twilight_qk")
    with on_device(dev):
        check(hip().tw_twilight_qk(ptr(q), G, R, D, ptr(packed), ptr(scale), ptr(minimum), _dt(scale), qe,
                                   packed.shape[1], ptr(plan_pages), ptr(plan_masks), ptr(plan_counts), plan_pages.stride(0),
                                   b0_pages, sink, block_size, qs, ptr(out), ptr(slot_u), ptr(page_rows),
                                   stream_handle(dev)), "twilight_qk")
    return out


def fused_affine_int4_qk(q: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, minimum: torch.Tensor,
                         positions: torch.Tensor, *, materialize: bool = False) -> torch.Tensor:
    """FP32 q . k~ (or the dequantized k~ itself with materialize=True) at the
    candidate positions (twilight_fused_qk.py:34-55).  q [G,R,D] fp32, packed
    [G,H,D/2] uint8, scale/minimum [G,H], positions [G,R,N] int64 in [0, H)."""
    if q.ndim != 3 or q.dtype != torch.float32:
        raise ValueError("expected an FP32 [G, R, D] query")
    g, r, d = q.shape
    h = packed.shape[1] if packed.ndim == 3 else -1
    n = positions.shape[-1]
    if packed.shape != (g, h, d // 2) or d not in (4, 8, 16, 32, 64, 128, 256):
        raise ValueError("packed must be [G, H, D/2] with a power-of-two head_dim in [4, 256]")
    if scale.shape != (g, h) or minimum.shape != (g, h) or positions.shape != (g, r, n):
        raise ValueError("incompatible affine INT4 metadata/positions")
    if packed.dtype != torch.uint8 or positions.dtype != torch.int64 or scale.dtype not in _KEY_DTYPES \
            or minimum.dtype != scale.dtype:
        raise ValueError("expected uint8 packed K, int64 positions and fp16/bf16/fp32 scale/minimum")
    _require_contiguous(q, packed, scale, minimum, positions, what="fused_affine_int4_qk")
    dev = _require_device(q, packed, scale, minimum, positions, what="fused_affine_int4_qk")
    out = torch.empty((g, r, n, d) if materialize else (g, r, n), device=dev, dtype=torch.float32)
    with on_device(dev):
        check(hip().tw_int4_qk_positions(ptr(q), g, r, d, ptr(packed), ptr(scale), ptr(minimum), _dt(scale), h, h,
                                         ptr(positions), n, 1.0, int(bool(materialize)), ptr(out),
                                         stream_handle(dev)), "fused_affine_int4_qk")
    return out


def twilight_max_candidates() -> int:
    """Largest candidate count per head (B0 pages x page size) the Twilight
    selection takes (tw_twilight_max_candidates)."""
    return int(hip().tw_twilight_max_candidates())


def twilight_select(
    logits: torch.Tensor,
    sel_pages: torch.Tensor,
    *,
    top_p: float,
    budget_mode: str,
    target_total: int = 0,
    rows: torch.Tensor,
    row_counts: torch.Tensor,
    desired: Optional[torch.Tensor] = None,
    allocated: Optional[torch.Tensor] = None,
    head_bits: Optional[torch.Tensor] = None,
    sink: int,
    recent: int,
    block_size: int,
    length: int,
    append_position: int = -1,
) -> None:
    """Top-p counts, (matched) budgets, token selection and the GQA union row
    list of one layer.  logits [G,R,N] from twilight_qk; sel_pages [G,R,b0]
    the stage-1 pages; rows [G, >=length+1] int32 and row_counts [G] int32
    receive the union (ascending, then append_position if >= 0); desired /
    allocated [G,R] int32 (optional) the counts; head_bits [G,R,ceil(N/32)]
    int32 (optional) each head's kept candidates as a bitmap.  budget_mode
    "given" takes allocated [G,R] as an input (every head keeps its
    top-allocated candidates; desired is not computed)."""
    modes = {"dynamic": 0, "matched": 1, "given": 2}
    if budget_mode not in modes:
        raise ValueError("budget_mode must be 'dynamic', 'matched' or 'given'")
    if budget_mode == "given" and allocated is None:
        raise ValueError("budget_mode 'given' needs the allocated counts")
    if logits.dtype != torch.float32 or logits.ndim != 3 or not logits.is_contiguous():
        raise ValueError("logits must be contiguous [G, R, N] fp32")
    G, R, N = logits.shape
    if sel_pages.dtype != torch.int32 or sel_pages.ndim != 3 or sel_pages.shape[:2] != (G, R) \
            or not sel_pages.is_contiguous():
        raise ValueError("sel_pages must be contiguous [G, R, b0] int32")
    b0 = sel_pages.shape[2]
    if b0 * block_size != N:
        raise ValueError("logits must hold b0_pages * block_size candidates per head")
    if rows.dtype != torch.int32 or rows.ndim != 2 or rows.shape[0] != G or rows.stride(1) != 1:
        raise ValueError("rows must be [G, stride] int32")
    if row_counts.dtype != torch.int32 or tuple(row_counts.shape) != (G,):
        raise ValueError("row_counts must be [G] int32")
    for t in (desired, allocated):
        if t is not None and (t.dtype != torch.int32 or tuple(t.shape) != (G, R) or not t.is_contiguous()):
            raise ValueError("desired/allocated must be contiguous [G, R] int32")
    if head_bits is not None and (head_bits.dtype != torch.int32 or tuple(head_bits.shape) != (G, R, (N + 31) // 32)
                                  or not head_bits.is_contiguous()):
        raise ValueError("head_bits must be contiguous [G, R, ceil(N/32)] int32")
    dev = _require_device(logits, sel_pages, rows, row_counts, desired, allocated, head_bits,
                          what="twilight_select")
    nbytes = hip().tw_twilight_select_workspace_size(G, R, N)
    ws = WORKSPACE.get(dev, "twilight_select", nbytes)
    with on_device(dev):
        check(hip().tw_twilight_select(ptr(logits), G, R, N, ptr(sel_pages), b0, float(top_p),
                                       modes[budget_mode], int(target_total), ptr(desired),
                                       ptr(allocated), ptr(head_bits), ptr(rows), ptr(row_counts), rows.stride(0), sink, recent,
                                       block_size, length, append_position, ptr(ws), ws.numel(),
                                       stream_handle(dev)), "twilight_select")


def twilight_select_ragged(
    logits: torch.Tensor,
    sel_pages: torch.Tensor,
    lengths: torch.Tensor,
    *,
    top_p: float,
    rows: torch.Tensor,
    row_counts: torch.Tensor,
    max_length: int,
    page_capacity: int,
    sink: int,
    recent: int,
    block_size: int,
    desired: Optional[torch.Tensor] = None,
    head_bits: Optional[torch.Tensor] = None,
) -> None:
    """twilight_select with dynamic budgets over groups of different lengths
    (lengths [G] int32 on the device, each <= max_length < rows.shape[1]):
    group g keeps min(ragged candidate pages, page_capacity, b0) B0 pages per
    head (sel_pages from quest_select_ragged, -1 beyond), and its union has
    no decode row (the attention takes cur_k/cur_v)."""
    if logits.dtype != torch.float32 or logits.ndim != 3 or not logits.is_contiguous():
        raise ValueError("logits must be contiguous [G, R, N] fp32")
    G, R, N = logits.shape
    if sel_pages.dtype != torch.int32 or sel_pages.ndim != 3 or sel_pages.shape[:2] != (G, R) \
            or not sel_pages.is_contiguous():
        raise ValueError("sel_pages must be contiguous [G, R, b0] int32")
    b0 = sel_pages.shape[2]
    if b0 * block_size != N:
        raise ValueError("logits must hold b0_pages * block_size candidates per head")
    if lengths.dtype != torch.int32 or tuple(lengths.shape) != (G,) or not lengths.is_contiguous():
        raise ValueError("lengths must be contiguous [G] int32")
    if rows.dtype != torch.int32 or rows.ndim != 2 or rows.shape[0] != G or rows.stride(1) != 1 \
            or rows.shape[1] <= max_length:
        raise ValueError("rows must be [G, > max_length] int32")
    if row_counts.dtype != torch.int32 or tuple(row_counts.shape) != (G,):
        raise ValueError("row_counts must be [G] int32")
    if desired is not None and (desired.dtype != torch.int32 or tuple(desired.shape) != (G, R)
                                or not desired.is_contiguous()):
        raise ValueError("desired must be contiguous [G, R] int32")
    if head_bits is not None and (head_bits.dtype != torch.int32 or tuple(head_bits.shape) != (G, R, (N + 31) // 32)
                                  or not head_bits.is_contiguous()):
        raise ValueError("head_bits must be contiguous [G, R, ceil(N/32)] int32")
    dev = _require_device(logits, sel_pages, lengths, rows, row_counts, desired, head_bits,
                          what="twilight_select_ragged")
    nbytes = hip().tw_twilight_select_workspace_size(G, R, N)
    ws = WORKSPACE.get(dev, "twilight_select", nbytes)
    with on_device(dev):
        check(hip().tw_twilight_select_ragged(ptr(logits), G, R, N, ptr(sel_pages), b0, float(top_p), ptr(desired),
                                              None, ptr(head_bits), ptr(rows), ptr(row_counts), rows.stride(0),
                                              sink, recent, block_size, ptr(lengths), int(max_length),
                                              int(page_capacity), ptr(ws), ws.numel(), stream_handle(dev)),
              "twilight_select_ragged")


def twilight_select_pages(
    logits: torch.Tensor,
    sel_pages: torch.Tensor,
    slot_u: torch.Tensor,
    page_rows: torch.Tensor,
    *,
    top_p: float,
    sink: int,
    recent: int,
    block_size: int,
    length: int = 0,
    lengths: Optional[torch.Tensor] = None,
    page_capacity: int = 0,
    desired: Optional[torch.Tensor] = None,
) -> None:
    """Top-p with dynamic budgets, each kept row published as a bit of its
    union page's row mask (page_rows, cleared by twilight_qk with the same
    slot_u) instead of a union row list.  lengths [G] int32 (device) for
    ragged groups, each clamped to `length` (their bound, as max_length of
    twilight_select_ragged); else every group has `length` tokens."""
    if logits.dtype != torch.float32 or logits.ndim != 3 or not logits.is_contiguous():
        raise ValueError("logits must be contiguous [G, R, N] fp32")
    G, R, N = logits.shape
    if sel_pages.dtype != torch.int32 or sel_pages.ndim != 3 or sel_pages.shape[:2] != (G, R) \
            or not sel_pages.is_contiguous():
        raise ValueError("sel_pages must be contiguous [G, R, b0] int32")
    b0 = sel_pages.shape[2]
    if b0 * block_size != N:
        raise ValueError("logits must hold b0_pages * block_size candidates per head")
    if slot_u.dtype != torch.int32 or tuple(slot_u.shape) != (G, R, b0) or not slot_u.is_contiguous():
        raise ValueError("slot_u must be contiguous [G, R, b0] int32")
    if page_rows.dtype != torch.int32 or page_rows.ndim != 2 or page_rows.shape[0] != G or page_rows.stride(1) != 1:
        raise ValueError("page_rows must be [G, stride] int32")
    if lengths is not None and (lengths.dtype != torch.int32 or tuple(lengths.shape) != (G,)
                                or not lengths.is_contiguous()):
        raise ValueError("lengths must be contiguous [G] int32")
    if desired is not None and (desired.dtype != torch.int32 or tuple(desired.shape) != (G, R)
                                or not desired.is_contiguous()):
        raise ValueError("desired must be contiguous [G, R] int32")
    dev = _require_device(logits, sel_pages, slot_u, page_rows, lengths, desired, what="twilight_select_pages")
    nbytes = hip().tw_twilight_select_workspace_size(G, R, N)
    ws = WORKSPACE.get(dev, "twilight_select", nbytes)
    with on_device(dev):
        check(hip().tw_twilight_select_pages(ptr(logits), G, R, N, ptr(sel_pages), b0, float(top_p), ptr(slot_u),
                                             ptr(page_rows), page_rows.stride(0), ptr(desired), sink, recent,
                                             block_size, int(length), ptr(lengths), int(page_capacity), ptr(ws),
                                             ws.numel(), stream_handle(dev)), "twilight_select_pages")


@functools.lru_cache(maxsize=None)
def _default_qk_scale(D: int) -> float:
    """1/sqrt(D) rounded to fp32 (the logit scale of the reference's INT4 QK)."""
    return float(torch.tensor(1.0 / math.sqrt(D), dtype=torch.float32))


def union_record_words(P: int) -> int:
    """int32 words of one KV group's Twilight union record over P scored
    pages: a page bitmap (whole 64-bit words), then 16-bit row masks two
    pages a word (16-byte padded)."""
    bits = 2 * ((P + 63) // 64)
    return ((bits + 3) & ~3) + ((((P + 1) // 2) + 3) & ~3)


def _check_int4_keys(packed: torch.Tensor, scale: torch.Tensor, minimum: torch.Tensor, G: int, D: int,
                     what: str) -> int:
    if packed.dtype != torch.uint8 or packed.ndim != 3 or packed.shape[0] != G or packed.shape[2] != D // 2:
        raise ValueError(f"{what}: packed must be [G, T, D/2] uint8")
    if packed.stride(2) != 1 or packed.stride(1) != D // 2 or packed.stride(0) % (D // 2):
        raise ValueError(f"{what}: packed rows must be contiguous")
    qe = packed.stride(0) // (D // 2)
    if scale.dtype not in _KEY_DTYPES or minimum.dtype != scale.dtype or scale.ndim != 2 or scale.shape[0] != G:
        raise ValueError(f"{what}: scale/minimum must be [G, T] in one key dtype")
    if scale.stride(1) != 1 or minimum.stride(1) != 1 or scale.stride(0) != qe or minimum.stride(0) != qe:
        raise ValueError(f"{what}: scale/minimum must share the packed entry stride")
    return qe


def twilight_select_fused(
    q: torch.Tensor,
    page_min: torch.Tensor,
    page_max: torch.Tensor,
    packed: torch.Tensor,
    scale: torch.Tensor,
    minimum: torch.Tensor,
    b0_pages: int,
    union_rec: torch.Tensor,
    *,
    top_p: float,
    sink: int,
    recent: int,
    block_size: int = 16,
    length: int = 0,
    lengths: Optional[torch.Tensor] = None,
    qk_scale: Optional[float] = None,
    desired: Optional[torch.Tensor] = None,
    sel_pages: Optional[torch.Tensor] = None,
    logits: Optional[torch.Tensor] = None,
    budget_mode: str = "dynamic",
    target_total: int = 0,
    allocated: Optional[torch.Tensor] = None,
    matched_fraction: float = 0.0,
    phase: int = 3,
) -> torch.Tensor:
    """The Twilight selection of a layer in two launches with dynamic budgets
    (Quest score + INT4 QK of every scored row; one block per head: B0 top-k,
    top-p, publish), or three with matched budgets (the head launch stops at
    the top-p counts; one block per head then forms the group's allocation
    towards target_total and keeps the head's top-allocated logits), written to each
    group's union record: union_rec [G, >= union_record_words(P)] int32 (row
    stride a multiple of 4, 16-byte aligned).  q [G, R, 128] fp32;
    page_min/page_max [G, >= P, 128] over the P scored pages (16-bit);
    packed/scale/minimum the INT4 keys.  lengths [G] int32 (device) for
    ragged groups, each clamped to `length`; else every group has `length`
    tokens.  Matched budgets take target_total rows per group for one
    length, or with lengths each group's own target from matched_fraction
    (the cache's fixed pages x 16 x R).  Returns desired [G, R] int32 (the
    top-p counts); sel_pages [G, R, b0_pages], logits [G, R, b0_pages * 16]
    and (matched) allocated [G, R] are optional outputs.  phase 1 runs the
    first launch alone (for timing it; the outputs are left as they were).
    More than 8 query heads per KV head run as sub-groups of at most 8; with
    matched budgets (at most 64 heads) they share one allocation over all R."""
    if phase not in (1, 3):
        raise ValueError("phase must be 1 (score + INT4 QK launch) or 3 (the selection)")
    if budget_mode not in ("dynamic", "matched"):
        raise ValueError("budget_mode must be 'dynamic' or 'matched'")
    matched = budget_mode == "matched"
    _check_score_inputs(q, page_min, page_max, "twilight_select_fused")
    G, R, D = q.shape
    P = page_min.shape[1]
    qe = _check_int4_keys(packed, scale, minimum, G, D, "twilight_select_fused")
    if not 1 <= b0_pages <= P:
        raise ValueError("b0_pages must be in [1, P]")
    if union_rec.dtype != torch.int32 or union_rec.ndim != 2 or union_rec.shape[0] != G \
            or union_rec.shape[1] < union_record_words(P) or union_rec.stride(1) != 1 or union_rec.stride(0) % 4 \
            or union_rec.data_ptr() % 16:
        raise ValueError("union_rec must be [G, >= union_record_words(P)] int32, rows 16-byte aligned")
    if lengths is not None and (lengths.dtype != torch.int32 or tuple(lengths.shape) != (G,)
                                or not lengths.is_contiguous()):
        raise ValueError("lengths must be contiguous [G] int32")
    dev = _require_device(q, page_min, page_max, packed, scale, minimum, union_rec, lengths, desired, sel_pages,
                          logits, allocated, what="twilight_select_fused")
    if desired is None:
        desired = torch.empty((G, R), dtype=torch.int32, device=dev)
    if matched:
        if lengths is not None:
            if not 0.0 < matched_fraction <= 1.0:
                raise ValueError("matched budgets over device lengths take 0 < matched_fraction <= 1")
            # each group's target is fixed(L_g) x 16 x R with fixed growing with
            # L_g, and its capacity min(b0, candidate pages) x 16 per head: past
            # b0 the reference's allocation raises (twilight_offload_cache.py:58-59),
            # so a launch whose longest group (at most `length`) would get there
            # is refused instead of clamped on the device
            sink_end = min(sink, length)
            recent_start = max(sink_end, length - max(0, recent - 1))
            eligible = recent_start - sink_end
            cand = min(eligible // block_size, P)
            fixed = min(cand, max(1, math.ceil(matched_fraction * eligible / block_size)))
            if cand > 0 and fixed > min(cand, b0_pages):
                raise ValueError(f"target_total is infeasible: the matched budget at length {length} is {fixed} "
                                 f"pages a head, past the {min(cand, b0_pages)} B0 pages")
        elif not R <= target_total <= R * b0_pages * block_size:
            raise ValueError("target_total must be in [R, R * b0_pages * block_size]")
        if sel_pages is None:  # the last launch reads the B0 pages
            sel_pages = torch.empty((G, R, b0_pages), dtype=torch.int32, device=dev)
    elif allocated is not None:
        raise ValueError("allocated is an output of matched budgets")
    for t, dt, shape in ((desired, torch.int32, (G, R)), (sel_pages, torch.int32, (G, R, b0_pages)),
                         (logits, torch.float32, (G, R, b0_pages * block_size)), (allocated, torch.int32, (G, R))):
        if t is not None and (t.dtype != dt or tuple(t.shape) != shape or not t.is_contiguous()):
            raise ValueError("twilight_select_fused output has the wrong dtype/shape")
    if R > 8:
        return _twilight_select_fused_wide(q, page_min, page_max, packed, scale, minimum, b0_pages, union_rec,
                                           top_p=top_p, sink=sink, recent=recent, block_size=block_size,
                                           length=length, lengths=lengths, qk_scale=qk_scale, desired=desired,
                                           sel_pages=sel_pages, logits=logits, budget_mode=budget_mode,
                                           target_total=target_total, allocated=allocated,
                                           matched_fraction=matched_fraction, phase=phase, dev=dev, qe=qe)
    qs = _default_qk_scale(D) if qk_scale is None else float(qk_scale)
    nbytes = hip().tw_twilight_select_fused_workspace_size(G, R, P, int(b0_pages))
    ws = WORKSPACE.get(dev, "twilight_fused", nbytes)
    with on_device(dev):
        if phase == 1:
            check(hip().tw_twilight_select_fused_phase(
                ptr(q), ptr(page_min), ptr(page_max), _dt(page_min), G, R, P, D, page_min.stride(0), ptr(packed),
                ptr(scale), ptr(minimum), qe, packed.shape[1], int(b0_pages), float(top_p), qs, sink, recent,
                block_size, ptr(lengths), int(length), ptr(sel_pages), ptr(logits), ptr(desired), ptr(union_rec),
                union_rec.stride(0), ptr(ws), ws.numel(), 1, stream_handle(dev)), "twilight_select_fused_phase")
        elif matched:
            check(hip().tw_twilight_select_fused_matched(
                ptr(q), ptr(page_min), ptr(page_max), _dt(page_min), G, R, P, D, page_min.stride(0), ptr(packed),
                ptr(scale), ptr(minimum), qe, packed.shape[1], int(b0_pages), float(top_p), qs, sink, recent,
                block_size, ptr(lengths), int(length), int(target_total), float(matched_fraction), ptr(sel_pages),
                ptr(logits), ptr(desired), ptr(allocated), ptr(union_rec), union_rec.stride(0), ptr(ws), ws.numel(),
                stream_handle(dev)),
                "twilight_select_fused_matched")
        else:
            check(hip().tw_twilight_select_fused(ptr(q), ptr(page_min), ptr(page_max), _dt(page_min), G, R, P, D,
                                                 page_min.stride(0), ptr(packed), ptr(scale), ptr(minimum), qe,
                                                 packed.shape[1], int(b0_pages), float(top_p), qs, sink, recent,
                                                 block_size, ptr(lengths), int(length), ptr(sel_pages), ptr(logits),
                                                 ptr(desired), ptr(union_rec), union_rec.stride(0), ptr(ws),
                                                 ws.numel(), stream_handle(dev)), "twilight_select_fused")
    return desired


def _twilight_select_fused_wide(q, page_min, page_max, packed, scale, minimum, b0_pages, union_rec, *, top_p, sink,
                                recent, block_size, length, lengths, qk_scale, desired, sel_pages, logits,
                                budget_mode, target_total, allocated, matched_fraction, phase, dev, qe):
    """twilight_select_fused for more than 8 query heads per KV head, as
    sub-groups of at most 8 (the outputs checked by the caller).  Dynamic
    budgets are each head's own, so the group's kept rows are the union of
    the sub-groups': the first sub-group writes union_rec, the others their
    own records ORed into it.  Matched budgets allocate over every head of the
    group: each sub-group's score + QK and head launches first (its top-p
    counts into its columns of desired), then each sub-group's allocation +
    top-allocated launch reads all of desired (tw_twilight_select_fused_matched_part)."""
    G, R, D = q.shape
    P = page_min.shape[1]
    matched = budget_mode == "matched"
    if phase != 3:
        raise ValueError("phase 1 takes at most 8 query heads per KV head")
    if matched and R > 64:
        raise ValueError("matched budgets over the fused selection take at most 64 query heads per KV head")
    chunks = head_chunks(R)
    extra = None
    if len(chunks) > 1:
        n_extra = len(chunks) - 1 if matched else 1
        extra = torch.empty((n_extra, G, union_rec.stride(0)), dtype=torch.int32, device=dev)

    def record(i):
        if i == 0:
            return union_rec
        return extra[i - 1 if matched else 0, :, :union_rec.shape[1]]

    if not matched:
        for i, (r0, r1) in enumerate(chunks):
            Rc = r1 - r0
            rec = record(i)
            d = torch.empty((G, Rc), dtype=torch.int32, device=dev)
            sp = None if sel_pages is None else torch.empty((G, Rc, b0_pages), dtype=torch.int32, device=dev)
            lg = None if logits is None else torch.empty((G, Rc, b0_pages * block_size), dtype=torch.float32,
                                                          device=dev)
            twilight_select_fused(q[:, r0:r1].contiguous(), page_min, page_max, packed, scale, minimum, b0_pages,
                                  rec, top_p=top_p, sink=sink, recent=recent, block_size=block_size, length=length,
                                  lengths=lengths, qk_scale=qk_scale, desired=d, sel_pages=sp, logits=lg)
            if i > 0:
                union_rec.bitwise_or_(rec)
            desired[:, r0:r1] = d
            if sp is not None:
                sel_pages[:, r0:r1] = sp
            if lg is not None:
                logits[:, r0:r1] = lg
        return desired
    qs = _default_qk_scale(D) if qk_scale is None else float(qk_scale)
    subs = []
    with on_device(dev):
        for part in (1, 2):
            for i, (r0, r1) in enumerate(chunks):
                Rc = r1 - r0
                if part == 1:
                    nbytes = hip().tw_twilight_select_fused_workspace_size(G, Rc, P, int(b0_pages))
                    subs.append(dict(
                        q=q[:, r0:r1].contiguous(), ws=WORKSPACE.get(dev, f"twilight_fused_sub{i}", nbytes),
                        d=torch.empty((G, Rc), dtype=torch.int32, device=dev),
                        sp=torch.empty((G, Rc, b0_pages), dtype=torch.int32, device=dev),
                        lg=None if logits is None else torch.empty((G, Rc, b0_pages * block_size),
                                                                   dtype=torch.float32, device=dev),
                        al=None if allocated is None else torch.empty((G, Rc), dtype=torch.int32, device=dev)))
                t = subs[i]
                rec = record(i)
                check(hip().tw_twilight_select_fused_matched_part(
                    ptr(t["q"]), ptr(page_min), ptr(page_max), _dt(page_min), G, Rc, P, D, page_min.stride(0),
                    ptr(packed), ptr(scale), ptr(minimum), qe, packed.shape[1], int(b0_pages), float(top_p), qs,
                    sink, recent, block_size, ptr(lengths), int(length), int(target_total), float(matched_fraction),
                    ptr(t["sp"]), ptr(t["lg"]), ptr(t["d"]), ptr(t["al"]), ptr(rec), union_rec.stride(0), part,
                    ptr(desired), R, r0, ptr(t["ws"]), t["ws"].numel(), stream_handle(dev)),
                    "twilight_select_fused_matched_part")
                if part == 1:
                    desired[:, r0:r1] = t["d"]
    for i, (r0, r1) in enumerate(chunks):
        t = subs[i]
        if i > 0:
            union_rec.bitwise_or_(record(i))
        if sel_pages is not None:
            sel_pages[:, r0:r1] = t["sp"]
        if logits is not None:
            logits[:, r0:r1] = t["lg"]
        if allocated is not None:
            allocated[:, r0:r1] = t["al"]
    return desired


# --------------------------------------------------------------- attention
def decode_attention_rows(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    rows: torch.Tensor,
    row_counts: torch.Tensor,
    max_rows: int,
    *,
    row_masks: Optional[torch.Tensor] = None,
    cur_k: Optional[torch.Tensor] = None,
    cur_v: Optional[torch.Tensor] = None,
    softmax_scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
    append_position: Optional[int] = None,
    metadata: Optional[dict] = None,
) -> torch.Tensor:
    """Sparse GQA decode attention reading K/V rows by position straight from
    the cache.  q [G,R,D]; k_cache/v_cache [G, Lmax, D] (the layer's entries,
    HBM or mapped pinned host); rows [G, stride] int32 positions; row_counts
    [G] int32; cur_k/cur_v [G, D] extra decode token.  With append_position
    (and cur_k/cur_v) the same launch also writes the decode token to that
    row of every entry -- an int, or an int32 [G] device tensor of per-group
    rows (rows outside the entry are skipped); the row list must not name
    it.  metadata (with the append; 16-bit K, D = 128): dict(sink=,
    page_min=, page_max= [G, pages, D], packed= [G, T, D/2], scale=,
    minimum= [G, T]) -- the launch also does update_page_metadata for the
    appended row (either pair may be left out).  Returns [G,R,D].

    More than 8 query heads per group run as sub-groups of at most 8 heads
    over the same rows (every head sees every row unless row_masks, which
    then limits R to 8); each sub-group's launch writes the same decode row."""
    if q.ndim != 3 or q.dtype not in _KEY_DTYPES:
        raise ValueError("q must be [G, R, D]")
    G, R, D = q.shape
    if R > 8:
        if row_masks is not None:
            raise ValueError("row_masks take at most 8 query heads per group")
        if out is None:
            out = torch.empty_like(q)
        for r0, r1 in head_chunks(R):
            out[:, r0:r1] = decode_attention_rows(
                q[:, r0:r1].contiguous(), k_cache, v_cache, rows, row_counts, max_rows, cur_k=cur_k, cur_v=cur_v,
                softmax_scale=softmax_scale, append_position=append_position, metadata=metadata)
        return out
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype or k_cache.shape != v_cache.shape:
        raise ValueError("K/V cache must match q's dtype and each other")
    if k_cache.ndim != 3 or k_cache.shape[0] != G or k_cache.shape[2] != D or k_cache.stride() != v_cache.stride():
        raise ValueError("K/V cache must be [G, Lmax, D]")
    if k_cache.stride(2) != 1 or k_cache.stride(1) != D or k_cache.stride(0) % D:
        raise ValueError("K/V cache rows must be contiguous")
    if rows.dtype != torch.int32 or rows.ndim != 2 or rows.shape[0] != G or rows.stride(1) != 1:
        raise ValueError("rows must be [G, stride] int32")
    if row_counts.dtype != torch.int32 or tuple(row_counts.shape) != (G,):
        raise ValueError("row_counts must be [G] int32")
    if (cur_k is None) != (cur_v is None):
        raise ValueError("cur_k and cur_v go together")
    if cur_k is not None and (cur_k.shape != (G, D) or cur_k.dtype != q.dtype or not cur_k.is_contiguous()
                              or not cur_v.is_contiguous() or cur_v.shape != cur_k.shape):
        raise ValueError("cur_k/cur_v must be contiguous [G, D] in q's dtype")
    dev = _require_device(q, rows, row_counts, row_masks, cur_k, cur_v, what="decode_attention")
    _require_contiguous(q, what="decode_attention")
    if out is None:
        out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    nbytes = hip().tw_decode_attention_workspace_size(G, R, D, max_rows)
    ws = WORKSPACE.get(dev, "decode_attention", nbytes)
    if append_position is not None:
        if cur_k is None:
            raise ValueError("append_position needs cur_k/cur_v")
        rows_dev = None
        if isinstance(append_position, torch.Tensor):
            if append_position.dtype != torch.int32 or tuple(append_position.shape) != (G,) \
                    or not append_position.is_contiguous() or append_position.device != q.device:
                raise ValueError("per-group append rows must be contiguous [G] int32 on q's device")
            rows_dev, pos = append_position, 0
        else:
            pos = int(append_position)
            if not 0 <= pos < k_cache.shape[1]:
                raise ValueError(f"append_position {pos} outside the cache rows [0, {k_cache.shape[1]})")
        md = dict(metadata or {})
        pmn, pmx, pk, qs, qm = (md.get(n) for n in ("page_min", "page_max", "packed", "scale", "minimum"))
        if pmn is not None and (pmx is None or pmn.ndim != 3 or pmn.shape[0] != G or pmn.shape[2] != D
                                or pmn.stride(2) != 1 or pmn.stride(1) != D or pmx.shape != pmn.shape
                                or pmx.stride() != pmn.stride() or pmn.dtype != q.dtype):
            raise ValueError("page_min/page_max must be [G, pages, D] with contiguous pages in q's dtype")
        if pk is not None and (qs is None or qm is None or pk.dtype != torch.uint8 or pk.ndim != 3
                               or pk.shape[0] != G or pk.shape[2] != D // 2 or pk.stride(2) != 1
                               or pk.stride(1) != D // 2 or qs.ndim != 2 or qs.shape[0] != G or qs.stride(1) != 1
                               or qm.stride() != qs.stride() or qs.dtype != q.dtype or qm.dtype != q.dtype
                               or pk.stride(0) // (D // 2) != qs.stride(0)):
            raise ValueError("packed [G, T, D/2] uint8 and scale/minimum [G, T] must match")
        if pmn is not None or pk is not None:
            _require_device(pmn, pmx, pk, qs, qm, what="decode_attention")
        with on_device(dev):
            check(hip().tw_decode_attention_rows_append(
                ptr(q), k_cache.data_ptr(), v_cache.data_ptr(), _dt(q), G, R, D, ptr(rows), ptr(row_masks),
                ptr(row_counts), rows.stride(0), k_cache.stride(0) // D, max_rows, ptr(cur_k), ptr(cur_v),
                pos, ptr(rows_dev), scale, int(md.get("sink", 0)), ptr(pmn), ptr(pmx),
                0 if pmn is None else pmn.stride(0), 0 if pmn is None else pmn.shape[1], ptr(pk), ptr(qs), ptr(qm),
                0 if qs is None else qs.stride(0), ptr(out), ptr(ws), ws.numel(), stream_handle(dev)),
                "decode_attention")
        return out
    with on_device(dev):
        check(hip().tw_decode_attention(ptr(q), k_cache.data_ptr(), v_cache.data_ptr(), _dt(q), G, R, D, ptr(rows),
                                        ptr(row_masks), ptr(row_counts), rows.stride(0), k_cache.stride(0) // D,
                                        None, 0, -1, max_rows, ptr(cur_k), ptr(cur_v), scale, ptr(out), ptr(ws),
                                        ws.numel(), stream_handle(dev)), "decode_attention")
    return out


def plan_max_rows(max_pages: int, *, sink: int, recent: int, block_size: int, length: int,
                  append_position: int = -1) -> int:
    """Bound on the rows of a union plan of at most max_pages pages."""
    sink_end = min(sink, length)
    recent_start = max(sink_end, length - max(0, recent - 1))
    return sink_end + max_pages * block_size + (length - recent_start) + (1 if append_position >= 0 else 0)


def decode_attention_pages(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    plan_pages: torch.Tensor,
    plan_counts: torch.Tensor,
    *,
    plan_masks: Optional[torch.Tensor] = None,
    max_pages: int,
    sink: int,
    recent: int,
    block_size: int,
    length: int,
    append_position: int = -1,
    cur_k: Optional[torch.Tensor] = None,
    cur_v: Optional[torch.Tensor] = None,
    softmax_scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
    phase: int = 3,
) -> torch.Tensor:
    """Sparse GQA decode attention over a union plan from quest_select: group
    g sees [0, sink_end) ++ its union pages (heads per plan_masks) ++ the
    recent window ++ the decode token.  q [G,R,D]; k_cache/v_cache [G, Lmax, D].
    The decode token is cache row append_position, or cur_k/cur_v [G, D] when
    given -- then they are also appended to row append_position of the cache
    in the same launch.  phase 1 runs only the split-K kernel, phase 2 only
    the merge of its partials (same arguments), 3 both.  Returns [G,R,D]."""
    if phase not in (1, 2, 3):
        raise ValueError("phase must be 1, 2 or 3")
    if q.ndim != 3 or q.dtype not in _KEY_DTYPES:
        raise ValueError("q must be [G, R, D]")
    G, R, D = q.shape
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype or k_cache.shape != v_cache.shape:
        raise ValueError("K/V cache must match q's dtype and each other")
    if k_cache.ndim != 3 or k_cache.shape[0] != G or k_cache.shape[2] != D or k_cache.stride() != v_cache.stride():
        raise ValueError("K/V cache must be [G, Lmax, D]")
    if k_cache.stride(2) != 1 or k_cache.stride(1) != D or k_cache.stride(0) % D:
        raise ValueError("K/V cache rows must be contiguous")
    if plan_pages.dtype != torch.int32 or plan_pages.ndim != 2 or plan_pages.shape[0] != G \
            or plan_pages.stride(1) != 1:
        raise ValueError("plan_pages must be [G, stride] int32")
    if plan_masks is not None and (plan_masks.dtype != torch.uint8 or plan_masks.shape != plan_pages.shape
                                   or plan_masks.stride() != plan_pages.stride()):
        raise ValueError("plan_masks must match plan_pages")
    if plan_counts.dtype != torch.int32 or tuple(plan_counts.shape) != (G,):
        raise ValueError("plan_counts must be [G] int32")
    if not 0 <= max_pages <= plan_pages.shape[1]:
        raise ValueError("max_pages must be within the plan width")
    if (cur_k is None) != (cur_v is None):
        raise ValueError("cur_k and cur_v go together")
    if cur_k is not None and (cur_k.shape != (G, D) or cur_k.dtype != q.dtype or cur_v.shape != cur_k.shape
                              or cur_v.dtype != q.dtype):
        raise ValueError("cur_k/cur_v must be [G, D] in q's dtype")
    if cur_k is not None and append_position >= k_cache.shape[1]:
        raise ValueError("append_position outside the cache")
    dev = _require_device(q, plan_pages, plan_masks, plan_counts, cur_k, cur_v, what="decode_attention_pages")
    if k_cache.is_cuda and k_cache.device != dev:
        raise ValueError("decode_attention_pages requires tensors on one device")
    kp, vp = _slab_source(k_cache, v_cache)
    _require_contiguous(q, cur_k, cur_v, what="decode_attention_pages")
    if out is None:
        out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    max_rows = plan_max_rows(max_pages, sink=sink, recent=recent, block_size=block_size, length=length,
                             append_position=append_position if cur_k is None else -1)
    max_rows += 0 if cur_k is None else 1
    nbytes = hip().tw_decode_attention_workspace_size(G, R, D, max_rows)
    ws = WORKSPACE.get(dev, "decode_attention", nbytes)
    with on_device(dev):
        check(hip().tw_decode_attention_pages_phase(ptr(q), kp, vp, _dt(q), G, R, D,
                                                    ptr(plan_pages), ptr(plan_masks), ptr(plan_counts),
                                                    plan_pages.stride(0), max_rows, k_cache.stride(0) // D, sink,
                                                    recent, block_size, length, append_position, ptr(cur_k),
                                                    ptr(cur_v), scale, ptr(out), ptr(ws), ws.numel(), int(phase),
                                                    stream_handle(dev)), "decode_attention_pages")
    return out


def _page_meta_args(page_min: Optional[torch.Tensor], page_max: Optional[torch.Tensor], G: int, D: int,
                    append: bool) -> tuple:
    """(ptr min, ptr max, entry stride, pages) of the fused page-metadata
    update; page_min/page_max [G, pages, D] views with contiguous pages."""
    if page_min is None and page_max is None:
        return None, None, 0, 0
    if page_min is None or page_max is None:
        raise ValueError("page_min and page_max go together")
    if not append:
        raise ValueError("the page metadata update follows the appended row (append=True)")
    if page_min.ndim != 3 or page_min.shape[0] != G or page_min.shape[2] != D or page_min.stride(2) != 1 \
            or page_min.stride(1) != D or page_max.shape != page_min.shape or page_max.stride() != page_min.stride():
        raise ValueError("page_min/page_max must be [G, pages, D] with contiguous pages")
    return ptr(page_min), ptr(page_max), page_min.stride(0), page_min.shape[1]


def decode_attention_pages_ragged(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    plan_pages: torch.Tensor,
    plan_counts: torch.Tensor,
    lengths: torch.Tensor,
    *,
    plan_masks: Optional[torch.Tensor] = None,
    max_pages: int,
    sink: int,
    recent: int,
    block_size: int = 16,
    append: bool = True,
    cur_k: Optional[torch.Tensor] = None,
    cur_v: Optional[torch.Tensor] = None,
    softmax_scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
    page_min: Optional[torch.Tensor] = None,
    page_max: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """decode_attention_pages over G groups of different lengths (lengths [G]
    int32 on the device): group g's window follows from its own length and
    its decode token is cur_k/cur_v[g] (appended at row lengths[g] when
    `append`), or the cache row lengths[g] (`append`, no cur_k), or none.
    16-bit K/V, D = 128, block_size 16.  k_cache/v_cache [G, Lmax, D] (HBM or
    pinned host).  With page_min/page_max [G, pages, D] the launch also does
    update_page_metadata_ragged's min/max of a page the appended row
    completes.  Returns [G, R, D]."""
    if q.ndim != 3 or q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("q must be [G, R, D] fp16/bf16")
    G, R, D = q.shape
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype or k_cache.shape != v_cache.shape \
            or k_cache.ndim != 3 or k_cache.shape[0] != G or k_cache.shape[2] != D \
            or k_cache.stride() != v_cache.stride() or k_cache.stride(2) != 1 or k_cache.stride(1) != D \
            or k_cache.stride(0) % D:
        raise ValueError("K/V cache must be row-contiguous [G, Lmax, D] in q's dtype")
    if plan_pages.dtype != torch.int32 or plan_pages.ndim != 2 or plan_pages.shape[0] != G \
            or plan_pages.stride(1) != 1:
        raise ValueError("plan_pages must be [G, stride] int32")
    if plan_masks is not None and (plan_masks.dtype != torch.uint8 or plan_masks.shape != plan_pages.shape
                                   or plan_masks.stride() != plan_pages.stride()):
        raise ValueError("plan_masks must match plan_pages")
    if plan_counts.dtype != torch.int32 or tuple(plan_counts.shape) != (G,):
        raise ValueError("plan_counts must be [G] int32")
    if lengths.dtype != torch.int32 or tuple(lengths.shape) != (G,) or not lengths.is_contiguous():
        raise ValueError("lengths must be contiguous [G] int32")
    if not 0 <= max_pages <= plan_pages.shape[1]:
        raise ValueError("max_pages must be within the plan width")
    if (cur_k is None) != (cur_v is None):
        raise ValueError("cur_k and cur_v go together")
    if cur_k is not None and (cur_k.shape != (G, D) or cur_k.dtype != q.dtype or cur_v.shape != cur_k.shape
                              or cur_v.dtype != q.dtype):
        raise ValueError("cur_k/cur_v must be [G, D] in q's dtype")
    dev = _require_device(q, plan_pages, plan_masks, plan_counts, lengths, cur_k, cur_v, page_min, page_max,
                          what="decode_attention_pages_ragged")
    meta = _page_meta_args(page_min, page_max, G, D, append)
    kp, vp = _slab_source(k_cache, v_cache)
    _require_contiguous(q, cur_k, cur_v, what="decode_attention_pages_ragged")
    if out is None:
        out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    max_rows = sink + max_pages * block_size + recent
    nbytes = hip().tw_decode_attention_workspace_size(G, R, D, max_rows)
    ws = WORKSPACE.get(dev, "decode_attention", nbytes)
    with on_device(dev):
        check(hip().tw_decode_attention_pages_ragged(ptr(q), kp, vp, _dt(q), G, R, D, ptr(plan_pages),
                                                     ptr(plan_masks), ptr(plan_counts), plan_pages.stride(0),
                                                     max_rows, k_cache.stride(0) // D, sink, recent, block_size,
                                                     ptr(lengths), int(bool(append)), ptr(cur_k), ptr(cur_v), scale,
                                                     *meta, ptr(out), ptr(ws), ws.numel(), stream_handle(dev)),
              "decode_attention_pages_ragged")
    return out


def decode_attention_pages_bits(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    sel_bits: torch.Tensor,
    P: int,
    *,
    max_pages: int,
    sink: int,
    recent: int,
    block_size: int = 16,
    lengths: Optional[torch.Tensor] = None,
    length: int = 0,
    append: bool = True,
    cur_k: Optional[torch.Tensor] = None,
    cur_v: Optional[torch.Tensor] = None,
    softmax_scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
    page_min: Optional[torch.Tensor] = None,
    page_max: Optional[torch.Tensor] = None,
    phase: int = 3,
) -> torch.Tensor:
    """decode_attention_pages(_ragged) with the union taken from the
    selection bitmaps of quest_select_bits ([G, R, words] int32 over P
    pages): the same tiles, in the same order, as the union plan gives.
    lengths ([G] int32, device) or length; the decode token is cur_k/cur_v
    (appended at the group's length when `append`).  max_pages bounds the
    union (R * k).  16-bit K/V, D = 128, block_size 16.  Returns [G, R, D]."""
    if phase not in (1, 2, 3):
        raise ValueError("phase must be 1, 2 or 3")
    if q.ndim != 3 or q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("q must be [G, R, D] fp16/bf16")
    G, R, D = q.shape
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype or k_cache.shape != v_cache.shape \
            or k_cache.ndim != 3 or k_cache.shape[0] != G or k_cache.shape[2] != D \
            or k_cache.stride() != v_cache.stride() or k_cache.stride(2) != 1 or k_cache.stride(1) != D \
            or k_cache.stride(0) % D:
        raise ValueError("K/V cache must be row-contiguous [G, Lmax, D] in q's dtype")
    if not 1 <= P <= 8192:
        raise ValueError("P must be in [1, 8192]")
    if sel_bits.dtype != torch.int32 or sel_bits.ndim != 3 or tuple(sel_bits.shape[:2]) != (G, R) \
            or sel_bits.shape[2] < sel_bits_words(P) or sel_bits.stride(2) != 1 \
            or sel_bits.stride(0) != R * sel_bits.stride(1) or sel_bits.stride(1) % 2 or sel_bits.data_ptr() % 8:
        raise ValueError("sel_bits must be [G, R, >= sel_bits_words(P)] int32 with 8-byte aligned rows")
    if lengths is not None and (lengths.dtype != torch.int32 or tuple(lengths.shape) != (G,)
                                or not lengths.is_contiguous()):
        raise ValueError("lengths must be contiguous [G] int32")
    if (cur_k is None) != (cur_v is None):
        raise ValueError("cur_k and cur_v go together")
    if cur_k is not None and (cur_k.shape != (G, D) or cur_k.dtype != q.dtype or cur_v.shape != cur_k.shape
                              or cur_v.dtype != q.dtype):
        raise ValueError("cur_k/cur_v must be [G, D] in q's dtype")
    if lengths is None and not 0 <= length < k_cache.shape[1]:
        raise ValueError("length outside the cache")
    dev = _require_device(q, sel_bits, lengths, cur_k, cur_v, page_min, page_max,
                          what="decode_attention_pages_bits")
    meta = _page_meta_args(page_min, page_max, G, D, append)
    kp, vp = _slab_source(k_cache, v_cache)
    _require_contiguous(q, cur_k, cur_v, what="decode_attention_pages_bits")
    if out is None:
        out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    max_rows = sink + max(0, max_pages) * block_size + recent
    nbytes = hip().tw_decode_attention_workspace_size(G, R, D, max_rows)
    ws = WORKSPACE.get(dev, "decode_attention", nbytes)
    with on_device(dev):
        check(hip().tw_decode_attention_pages_bits(ptr(q), kp, vp, _dt(q), G, R, D, ptr(sel_bits),
                                                   sel_bits.stride(1), P, max_rows, k_cache.stride(0) // D, sink,
                                                   recent, block_size, ptr(lengths), int(length),
                                                   int(bool(append)), ptr(cur_k), ptr(cur_v), scale, *meta,
                                                   ptr(out), ptr(ws), ws.numel(), int(phase), stream_handle(dev)),
              "decode_attention_pages_bits")
    return out


def decode_attention_page_rows(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    plan_pages: torch.Tensor,
    plan_counts: torch.Tensor,
    page_rows: torch.Tensor,
    *,
    max_pages: int,
    sink: int,
    recent: int,
    block_size: int = 16,
    lengths: Optional[torch.Tensor] = None,
    length: int = 0,
    append: bool = True,
    cur_k: Optional[torch.Tensor] = None,
    cur_v: Optional[torch.Tensor] = None,
    softmax_scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
    page_min: Optional[torch.Tensor] = None,
    page_max: Optional[torch.Tensor] = None,
    packed: Optional[torch.Tensor] = None,
    scale: Optional[torch.Tensor] = None,
    minimum: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """The Twilight union attention over page rows: every head attends the
    kept rows of the B0 union pages (page_rows from twilight_select_pages,
    int32 shaped like plan_pages), the sink and recent windows and the decode
    token.  lengths [G] int32 (device) for ragged groups, else every group has
    `length` tokens.  append / cur_k / cur_v / page_min / page_max as
    decode_attention_pages_ragged; packed [G, T, D/2] with scale / minimum
    [G, T] (16-bit) also get the appended row's INT4 code.  16-bit K/V,
    D = 128, block_size 16.  Returns [G, R, D]."""
    if q.ndim != 3 or q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("q must be [G, R, D] fp16/bf16")
    G, R, D = q.shape
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype or k_cache.shape != v_cache.shape \
            or k_cache.ndim != 3 or k_cache.shape[0] != G or k_cache.shape[2] != D \
            or k_cache.stride() != v_cache.stride() or k_cache.stride(2) != 1 or k_cache.stride(1) != D \
            or k_cache.stride(0) % D:
        raise ValueError("K/V cache must be row-contiguous [G, Lmax, D] in q's dtype")
    if plan_pages.dtype != torch.int32 or plan_pages.ndim != 2 or plan_pages.shape[0] != G \
            or plan_pages.stride(1) != 1:
        raise ValueError("plan_pages must be [G, stride] int32")
    if page_rows.dtype != torch.int32 or page_rows.shape != plan_pages.shape or page_rows.stride() != plan_pages.stride():
        raise ValueError("page_rows must be int32 shaped and strided like plan_pages")
    if plan_counts.dtype != torch.int32 or tuple(plan_counts.shape) != (G,):
        raise ValueError("plan_counts must be [G] int32")
    if lengths is not None and (lengths.dtype != torch.int32 or tuple(lengths.shape) != (G,)
                                or not lengths.is_contiguous()):
        raise ValueError("lengths must be contiguous [G] int32")
    if lengths is None and not 0 <= int(length) < k_cache.shape[1]:
        raise ValueError("length must leave the decode row inside the cache")
    if not 0 <= max_pages <= plan_pages.shape[1]:
        raise ValueError("max_pages must be within the plan width")
    if (cur_k is None) != (cur_v is None):
        raise ValueError("cur_k and cur_v go together")
    if cur_k is not None and (cur_k.shape != (G, D) or cur_k.dtype != q.dtype or cur_v.shape != cur_k.shape
                              or cur_v.dtype != q.dtype):
        raise ValueError("cur_k/cur_v must be [G, D] in q's dtype")
    if packed is not None and (scale is None or minimum is None or cur_k is None or not append
                               or packed.dtype != torch.uint8 or packed.ndim != 3 or packed.shape[0] != G
                               or packed.shape[2] != D // 2 or packed.stride(2) != 1 or packed.stride(1) != D // 2
                               or scale.ndim != 2 or scale.shape[0] != G or scale.stride(1) != 1
                               or minimum.stride() != scale.stride() or scale.dtype != q.dtype
                               or minimum.dtype != q.dtype or packed.stride(0) // (D // 2) != scale.stride(0)):
        raise ValueError("packed [G, T, D/2] uint8 and scale/minimum [G, T] must match (with cur_k and append)")
    dev = _require_device(q, plan_pages, plan_counts, page_rows, lengths, cur_k, cur_v, page_min, page_max, packed,
                          scale, minimum, what="decode_attention_page_rows")
    meta = _page_meta_args(page_min, page_max, G, D, append)
    kp, vp = _slab_source(k_cache, v_cache)
    _require_contiguous(q, cur_k, cur_v, what="decode_attention_page_rows")
    if out is None:
        out = torch.empty_like(q)
    sc = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    max_rows = sink + max_pages * block_size + recent
    nbytes = hip().tw_decode_attention_workspace_size(G, R, D, max_rows)
    ws = WORKSPACE.get(dev, "decode_attention", nbytes)
    with on_device(dev):
        check(hip().tw_decode_attention_page_rows(ptr(q), kp, vp, _dt(q), G, R, D, ptr(plan_pages), ptr(plan_counts),
                                                  ptr(page_rows), plan_pages.stride(0), max_rows,
                                                  k_cache.stride(0) // D, sink, recent, block_size, ptr(lengths),
                                                  int(length), int(bool(append)), ptr(cur_k), ptr(cur_v), sc, *meta,
                                                  ptr(packed), ptr(scale), ptr(minimum),
                                                  0 if scale is None else scale.stride(0), ptr(out), ptr(ws),
                                                  ws.numel(), stream_handle(dev)), "decode_attention_page_rows")
    return out


def decode_attention_union(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    union_rec: torch.Tensor,
    P: int,
    *,
    max_pages: int,
    sink: int,
    recent: int,
    block_size: int = 16,
    lengths: Optional[torch.Tensor] = None,
    length: int = 0,
    append: bool = True,
    cur_k: Optional[torch.Tensor] = None,
    cur_v: Optional[torch.Tensor] = None,
    softmax_scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
    page_min: Optional[torch.Tensor] = None,
    page_max: Optional[torch.Tensor] = None,
    packed: Optional[torch.Tensor] = None,
    scale: Optional[torch.Tensor] = None,
    minimum: Optional[torch.Tensor] = None,
    phase: int = 3,
    resident: Optional["ResidentPages"] = None,
) -> torch.Tensor:
    """The Twilight union attention from the union records of
    twilight_select_fused over P pages: every head attends the kept rows of
    the union pages, the sink and recent windows and the decode token.
    max_pages bounds a group's union pages (min(P, R * b0_pages)); the other
    arguments as decode_attention_page_rows.  More than 8 query heads per
    group run as sub-groups of at most 8 over the same record.  resident
    (R <= 8; a ResidentPages over this launch's groups, slots <= 65535): the
    previous-token resident cache, row by row -- a kept row the previous
    step kept too is read from HBM -- with its sink/recent windows, and its
    stats counting (hit rows, union rows).  Returns [G, R, D]."""
    if phase not in (1, 2, 3):
        raise ValueError("phase must be 1, 2 or 3")
    if q.ndim != 3 or q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("q must be [G, R, D] fp16/bf16")
    G, R, D = q.shape
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype or k_cache.shape != v_cache.shape \
            or k_cache.ndim != 3 or k_cache.shape[0] != G or k_cache.shape[2] != D \
            or k_cache.stride() != v_cache.stride() or k_cache.stride(2) != 1 or k_cache.stride(1) != D \
            or k_cache.stride(0) % D:
        raise ValueError("K/V cache must be row-contiguous [G, Lmax, D] in q's dtype")
    if not 1 <= P <= 8192:
        raise ValueError("P must be in [1, 8192]")
    if union_rec.dtype != torch.int32 or union_rec.ndim != 2 or union_rec.shape[0] != G \
            or union_rec.shape[1] < union_record_words(P) or union_rec.stride(1) != 1 or union_rec.stride(0) % 4 \
            or union_rec.data_ptr() % 16:
        raise ValueError("union_rec must be [G, >= union_record_words(P)] int32, rows 16-byte aligned")
    if lengths is not None and (lengths.dtype != torch.int32 or tuple(lengths.shape) != (G,)
                                or not lengths.is_contiguous()):
        raise ValueError("lengths must be contiguous [G] int32")
    if lengths is None and not 0 <= int(length) < k_cache.shape[1]:
        raise ValueError("length must leave the decode row inside the cache")
    if (cur_k is None) != (cur_v is None):
        raise ValueError("cur_k and cur_v go together")
    if cur_k is not None and (cur_k.shape != (G, D) or cur_k.dtype != q.dtype or cur_v.shape != cur_k.shape
                              or cur_v.dtype != q.dtype):
        raise ValueError("cur_k/cur_v must be [G, D] in q's dtype")
    if packed is not None and (scale is None or minimum is None or cur_k is None or not append
                               or packed.dtype != torch.uint8 or packed.ndim != 3 or packed.shape[0] != G
                               or packed.shape[2] != D // 2 or packed.stride(2) != 1 or packed.stride(1) != D // 2
                               or scale.ndim != 2 or scale.shape[0] != G or scale.stride(1) != 1
                               or minimum.stride() != scale.stride() or scale.dtype != q.dtype
                               or minimum.dtype != q.dtype or packed.stride(0) // (D // 2) != scale.stride(0)):
        raise ValueError("packed [G, T, D/2] uint8 and scale/minimum [G, T] must match (with cur_k and append)")
    if resident is not None:
        if R > 8:
            raise ValueError("the resident cache takes at most 8 query heads per KV head")
        if resident.slots > 0xffff:
            raise ValueError("the resident cache over a union record takes at most 65535 slots")
        _check_resident(resident, q, G, D, sink, recent)
    res = () if resident is None else (resident.k, resident.v, resident.map, resident.stats, resident.win_k,
                                       resident.win_v, resident.win_state)
    dev = _require_device(q, union_rec, lengths, cur_k, cur_v, page_min, page_max, packed, scale, minimum, *res,
                          what="decode_attention_union")
    meta = _page_meta_args(page_min, page_max, G, D, append)
    kp, vp = _slab_source(k_cache, v_cache)
    _require_contiguous(q, cur_k, cur_v, what="decode_attention_union")
    if out is None:
        out = torch.empty_like(q)
    if R > 8:
        # sub-groups of at most 8 heads over the same record (every head
        # attends every kept row); each launch writes the same decode row and
        # completes the same metadata
        if phase != 3:
            raise ValueError("phases 1 and 2 take at most 8 query heads per KV head")
        for r0, r1 in head_chunks(R):
            out[:, r0:r1] = decode_attention_union(
                q[:, r0:r1].contiguous(), k_cache, v_cache, union_rec, P, max_pages=max_pages, sink=sink,
                recent=recent, block_size=block_size, lengths=lengths, length=length, append=append, cur_k=cur_k,
                cur_v=cur_v, softmax_scale=softmax_scale, page_min=page_min, page_max=page_max, packed=packed,
                scale=scale, minimum=minimum)
        return out
    sc = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    max_rows = sink + max(0, max_pages) * block_size + recent
    nbytes = hip().tw_decode_attention_workspace_size(G, R, D, max_rows)
    ws = WORKSPACE.get(dev, "decode_attention", nbytes)
    with on_device(dev):
        if resident is None:
            check(hip().tw_decode_attention_union(
                ptr(q), kp, vp, _dt(q), G, R, D, ptr(union_rec), union_rec.stride(0), P, max_rows,
                k_cache.stride(0) // D, sink, recent, block_size, ptr(lengths), int(length), int(bool(append)),
                ptr(cur_k), ptr(cur_v), sc, *meta, ptr(packed), ptr(scale), ptr(minimum),
                0 if scale is None else scale.stride(0), ptr(out), ptr(ws), ws.numel(), int(phase),
                stream_handle(dev)), "decode_attention_union")
        else:
            wk = resident.win_k
            check(hip().tw_decode_attention_union_resident(
                ptr(q), kp, vp, _dt(q), G, R, D, ptr(union_rec), union_rec.stride(0), P, max_rows,
                k_cache.stride(0) // D, sink, recent, block_size, ptr(lengths), int(length), int(bool(append)),
                ptr(cur_k), ptr(cur_v), sc, ptr(resident.k), ptr(resident.v), ptr(resident.map), resident.slots,
                resident.pages, ptr(resident.stats), ptr(wk), ptr(resident.win_v), ptr(resident.win_state),
                resident.ring if wk is not None else 0, *meta, ptr(packed), ptr(scale), ptr(minimum),
                0 if scale is None else scale.stride(0), ptr(out), ptr(ws), ws.numel(), int(phase),
                stream_handle(dev)), "decode_attention_union_resident")
    return out


class ResidentPages:
    """HBM resident page cache of G groups (one layer's entries) for a slab
    in host memory: K/V buffers [G, 2, slots, 16, D], the page map [G, pages]
    int64 (-1 = never stored) and stats [G, 2] (hit pages, union pages).
    With sink/recent given, the resident windows too: win_k/win_v [G, sink +
    ring, D] (the sink rows, then a ring of the latest `ring` rows, ring the
    smallest power of two >= recent: recent - 1 history rows and the decode
    row) and win_state [G, 2] int32 (zeroed:
    nothing stored yet)."""

    def __init__(self, groups: int, slots: int, pages: int, head_dim: int, dtype: torch.dtype,
                 device: torch.device, sink: int = 0, recent: int = 0) -> None:
        self.k = torch.empty((groups, 2, slots, 16, head_dim), dtype=dtype, device=device)
        self.v = torch.empty_like(self.k)
        self.map = torch.full((groups, pages), -1, dtype=torch.int64, device=device)
        self.stats = torch.zeros((groups, 2), dtype=torch.int64, device=device)
        self.slots, self.pages = slots, pages
        self.sink = sink
        self.ring = 1 << (max(recent, 1) - 1).bit_length() if sink + recent > 0 else 0
        self.win_k = self.win_v = self.win_state = None
        if self.ring > 0:
            self.win_k = torch.empty((groups, sink + self.ring, head_dim), dtype=dtype, device=device)
            self.win_v = torch.empty_like(self.win_k)
            self.win_state = torch.zeros((groups, 2), dtype=torch.int32, device=device)

    def view(self, g0: int, n: int) -> "ResidentPages":
        out = ResidentPages.__new__(ResidentPages)
        out.k, out.v = self.k[g0:g0 + n], self.v[g0:g0 + n]
        out.map, out.stats = self.map[g0:g0 + n], self.stats[g0:g0 + n]
        out.slots, out.pages = self.slots, self.pages
        out.sink, out.ring = self.sink, self.ring
        out.win_k = out.win_v = out.win_state = None
        if self.win_k is not None:
            out.win_k, out.win_v = self.win_k[g0:g0 + n], self.win_v[g0:g0 + n]
            out.win_state = self.win_state[g0:g0 + n]
        return out


def _check_resident(resident: "ResidentPages", q: torch.Tensor, G: int, D: int, sink: int, recent: int) -> None:
    rk, rv, rm, rs = resident.k, resident.v, resident.map, resident.stats
    if rk.dtype != q.dtype or tuple(rk.shape) != (G, 2, resident.slots, 16, D) or not rk.is_contiguous() \
            or rv.shape != rk.shape or not rv.is_contiguous() or rm.dtype != torch.int64 \
            or tuple(rm.shape) != (G, resident.pages) or not rm.is_contiguous() \
            or tuple(rs.shape) != (G, 2) or not rs.is_contiguous():
        raise ValueError("resident buffers do not match the launch")
    wk, wv, wst = resident.win_k, resident.win_v, resident.win_state
    if wk is not None and (resident.sink != sink or resident.ring < recent or wk.dtype != q.dtype
                           or tuple(wk.shape) != (G, sink + resident.ring, D) or not wk.is_contiguous()
                           or wv.shape != wk.shape or not wv.is_contiguous() or wst.dtype != torch.int32
                           or tuple(wst.shape) != (G, 2) or not wst.is_contiguous()):
        raise ValueError("resident windows do not match the launch (sink, recent, dtype, shape)")


def decode_attention_pages_resident(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    plan_pages: torch.Tensor,
    plan_counts: torch.Tensor,
    resident: ResidentPages,
    *,
    lengths: Optional[torch.Tensor] = None,
    length: int = 0,
    plan_masks: Optional[torch.Tensor] = None,
    max_pages: int,
    sink: int,
    recent: int,
    block_size: int = 16,
    append: bool = True,
    cur_k: Optional[torch.Tensor] = None,
    cur_v: Optional[torch.Tensor] = None,
    softmax_scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
    page_min: Optional[torch.Tensor] = None,
    page_max: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """decode_attention_pages (lengths None: one `length`) or its ragged form
    (lengths [G] int32 on the device), with union pages kept in an HBM
    resident page cache: pages the previous step stored are read from HBM,
    the rest from the slab, and every union page read is stored for the next
    step.  With resident windows (a ResidentPages built with sink/recent),
    the sink rows and the recent window come from HBM once stored, and the
    decode row joins the ring every step.  16-bit K/V, D = 128, block_size
    16.  page_min/page_max as in decode_attention_pages_ragged.  Returns
    [G, R, D]."""
    if q.ndim != 3 or q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("q must be [G, R, D] fp16/bf16")
    G, R, D = q.shape
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype or k_cache.shape != v_cache.shape \
            or k_cache.ndim != 3 or k_cache.shape[0] != G or k_cache.shape[2] != D \
            or k_cache.stride() != v_cache.stride() or k_cache.stride(2) != 1 or k_cache.stride(1) != D \
            or k_cache.stride(0) % D:
        raise ValueError("K/V cache must be row-contiguous [G, Lmax, D] in q's dtype")
    if plan_pages.dtype != torch.int32 or plan_pages.ndim != 2 or plan_pages.shape[0] != G \
            or plan_pages.stride(1) != 1:
        raise ValueError("plan_pages must be [G, stride] int32")
    if plan_masks is not None and (plan_masks.dtype != torch.uint8 or plan_masks.shape != plan_pages.shape
                                   or plan_masks.stride() != plan_pages.stride()):
        raise ValueError("plan_masks must match plan_pages")
    if plan_counts.dtype != torch.int32 or tuple(plan_counts.shape) != (G,):
        raise ValueError("plan_counts must be [G] int32")
    if lengths is not None and (lengths.dtype != torch.int32 or tuple(lengths.shape) != (G,)
                                or not lengths.is_contiguous()):
        raise ValueError("lengths must be contiguous [G] int32")
    rk, rv, rm, rs = resident.k, resident.v, resident.map, resident.stats
    _check_resident(resident, q, G, D, sink, recent)
    wk, wv, wst = resident.win_k, resident.win_v, resident.win_state
    if not 0 <= max_pages <= plan_pages.shape[1]:
        raise ValueError("max_pages must be within the plan width")
    if (cur_k is None) != (cur_v is None):
        raise ValueError("cur_k and cur_v go together")
    if cur_k is not None and (cur_k.shape != (G, D) or cur_k.dtype != q.dtype or cur_v.shape != cur_k.shape
                              or cur_v.dtype != q.dtype):
        raise ValueError("cur_k/cur_v must be [G, D] in q's dtype")
    dev = _require_device(q, plan_pages, plan_masks, plan_counts, lengths, cur_k, cur_v, rk, rv, rm, rs, page_min,
                          page_max, what="decode_attention_pages_resident")
    meta = _page_meta_args(page_min, page_max, G, D, append)
    kp, vp = _slab_source(k_cache, v_cache)
    _require_contiguous(q, cur_k, cur_v, what="decode_attention_pages_resident")
    if out is None:
        out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    max_rows = sink + max_pages * block_size + recent
    nbytes = hip().tw_decode_attention_workspace_size(G, R, D, max_rows)
    ws = WORKSPACE.get(dev, "decode_attention", nbytes)
    with on_device(dev):
        check(hip().tw_decode_attention_pages_resident(
            ptr(q), kp, vp, _dt(q), G, R, D, ptr(plan_pages), ptr(plan_masks), ptr(plan_counts),
            plan_pages.stride(0), max_rows, k_cache.stride(0) // D, sink, recent, block_size, ptr(lengths),
            int(length), int(bool(append)), ptr(cur_k), ptr(cur_v), scale, ptr(rk), ptr(rv), ptr(rm),
            resident.slots, resident.pages, ptr(rs), ptr(wk), ptr(wv), ptr(wst), resident.ring if wk is not None else 0,
            *meta, ptr(out), ptr(ws), ws.numel(), stream_handle(dev)),
            "decode_attention_pages_resident")
    return out


def decode_attention_varlen(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_k: int,
    *,
    softmax_scale: Optional[float] = None,
    window_left: int = -1,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Varlen decode attention with one query token per sequence (the
    flash_attn_varlen_func call of mp.py:40-52 at max_seqlen_q == 1).
    q [B, Hq, D], k/v [total_k, Hk, D], cu_seqlens_k [B+1] int32."""
    if q.ndim != 3 or k.ndim != 3 or v.shape != k.shape:
        raise ValueError("expected q [B, Hq, D] and k/v [total_k, Hk, D]")
    B, Hq, D = q.shape
    Hk = k.shape[1]
    if k.shape[2] != D or Hq % Hk:
        raise ValueError("head_dim mismatch or Hq not a multiple of Hk")
    if q.dtype not in _KEY_DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q/k/v dtypes must match (fp16/bf16/fp32)")
    if cu_seqlens_k.dtype != torch.int32 or tuple(cu_seqlens_k.shape) != (B + 1,):
        raise ValueError("cu_seqlens_k must be [B+1] int32")
    dev = _require_device(q, k, v, cu_seqlens_k, what="decode_attention_varlen")
    _require_contiguous(q, k, v, cu_seqlens_k, what="decode_attention_varlen")
    R = Hq // Hk
    G = B * Hk
    if out is None:
        out = torch.empty_like(q)
    if R > 8:
        # sub-groups of at most 8 query heads per KV head over the same keys
        qv, ov = q.view(B, Hk, R, D), out.view(B, Hk, R, D)
        for r0, r1 in head_chunks(R):
            res = decode_attention_varlen(qv[:, :, r0:r1].reshape(B, Hk * (r1 - r0), D).contiguous(), k, v,
                                          cu_seqlens_k, max_seqlen_k, softmax_scale=softmax_scale,
                                          window_left=window_left)
            ov[:, :, r0:r1] = res.view(B, Hk, r1 - r0, D)
        return out
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    max_rows = int(max_seqlen_k)
    if window_left >= 0:
        max_rows = min(max_rows, window_left + 1)
    nbytes = hip().tw_decode_attention_workspace_size(G, R, D, max_rows)
    ws = WORKSPACE.get(dev, "decode_attention", nbytes)
    with on_device(dev):
        check(hip().tw_decode_attention(ptr(q), k.data_ptr(), v.data_ptr(), _dt(q), G, R, D, None, None, None, 0, 0,
                                        ptr(cu_seqlens_k), Hk, int(window_left), max_rows, None, None, scale,
                                        ptr(out), ptr(ws), ws.numel(), stream_handle(dev)), "decode_attention_varlen")
    return out


# ------------------------------------------------------------ row movement
_DEVICE_ALIAS: dict[int, int] = {}


def host_device_pointer(t: torch.Tensor) -> int:
    """Device address of a pinned host tensor's data (zero-copy access).  The
    mapping is looked up for the start of the tensor's pinned allocation (its
    storage) and offset to the view."""
    if t.is_cuda or not t.is_pinned():
        raise ValueError("zero-copy source must be pinned host memory")
    base = t.untyped_storage().data_ptr()
    dev = _DEVICE_ALIAS.get(base)
    if dev is None:
        out = _native.ctypes.c_void_p()
        check(hip().tw_host_device_pointer(base, _native.ctypes.byref(out)), "host_device_pointer")
        dev = int(out.value)
        _DEVICE_ALIAS[base] = dev
    return dev + (t.data_ptr() - base)


def gather_rows(
    src_k: torch.Tensor,
    src_v: torch.Tensor,
    src_rows: torch.Tensor,
    dst_k: torch.Tensor,
    dst_v: torch.Tensor,
    dst_rows: Optional[torch.Tensor] = None,
    *,
    error_flag: Optional[torch.Tensor] = None,
    device: Optional[torch.device] = None,
) -> None:
    """dst[dst_rows[i]] = src[src_rows[i]] for K and V (bit-exact).

    src_k/src_v: [rows, D] on the device, or pinned host tensors (read
    zero-copy through their mapped device address).  dst_k/dst_v: matching
    contiguous [..., D] buffers of capacity numel // D rows.  src_rows/dst_rows:
    int64 device tensors (without dst_rows, row i goes to row i, and
    len(src_rows) must fit the destination).  A pair with an out-of-range
    source or destination row is skipped and flagged in error_flag (int32
    device scalar)."""
    if src_k.shape != src_v.shape or src_k.dtype != src_v.dtype or src_k.ndim != 2:
        raise ValueError("src_k/src_v must be matching [rows, D]")
    if dst_k.dtype != src_k.dtype or dst_v.dtype != src_k.dtype or dst_k.shape[-1] != src_k.shape[-1]:
        raise ValueError("destination must match the source dtype and row width")
    if dst_k.shape != dst_v.shape:
        raise ValueError("dst_k/dst_v must match")
    dst_capacity = dst_k.numel() // src_k.shape[1]
    if dst_rows is None and src_rows.numel() > dst_capacity:
        raise ValueError(f"{src_rows.numel()} rows do not fit a destination of {dst_capacity} rows")
    _require_contiguous(src_k, src_v, dst_k, dst_v, src_rows, dst_rows, what="gather_rows")
    if src_rows.dtype != torch.int64 or (dst_rows is not None and (dst_rows.dtype != torch.int64
                                                                   or dst_rows.shape != src_rows.shape)):
        raise ValueError("row indices must be int64")
    dev = _require_device(dst_k, dst_v, src_rows, dst_rows, error_flag, what="gather_rows")
    if src_k.is_cuda:
        sk, sv = src_k.data_ptr(), src_v.data_ptr()
    else:
        sk, sv = host_device_pointer(src_k), host_device_pointer(src_v)
    D = src_k.shape[1]
    with on_device(dev):
        check(hip().tw_gather_rows(sk, sv, src_k.shape[0], ptr(src_rows), ptr(dst_rows), src_rows.numel(),
                                   dst_capacity, D, src_k.element_size(), ptr(dst_k), ptr(dst_v), ptr(error_flag),
                                   stream_handle(dev)), "gather_rows")


def _slab_source(src_k: torch.Tensor, src_v: torch.Tensor) -> tuple[int, int]:
    """Device addresses of a K/V source: HBM tensors, or pinned host tensors
    read zero-copy through their mapped device address."""
    if src_k.is_cuda != src_v.is_cuda:
        raise ValueError("K and V sources must live in the same memory")
    if src_k.is_cuda:
        return src_k.data_ptr(), src_v.data_ptr()
    return host_device_pointer(src_k), host_device_pointer(src_v)


def gather_union(
    src_k: torch.Tensor,
    src_v: torch.Tensor,
    rows: torch.Tensor,
    row_counts: torch.Tensor,
    cur_k: torch.Tensor,
    cur_v: torch.Tensor,
    dst_k: torch.Tensor,
    dst_v: torch.Tensor,
    cu_seqlens: torch.Tensor,
    *,
    entry_row0: int,
    entry_row_step: int,
    max_count: int,
    error_flag: Optional[torch.Tensor] = None,
    resident: Optional[dict] = None,
) -> None:
    """Pack each group's union rows, then its decode token, back to back
    (the varlen K/V of the GQA group path) and write cu_seqlens [G+1].

    src_k/src_v: the slab planes [rows, D] (HBM or pinned host); group g's
    source rows are entry_row0 + g*entry_row_step + rows[g, i]; rows [G,
    stride] int32 and row_counts [G] int32 on the device; cur_k/cur_v [G, D];
    dst_k/dst_v [capacity, D].  resident (the previous-token resident cache):
    dict(map= [G, positions] int64 (-1 at first), epoch= this step's history
    length, prev_k=, prev_v= the previous step's packed output, prev_cu= its
    cu_seqlens, stats= [2] int64 or None): rows the previous step packed are
    copied from there, and the map then names this step's rows."""
    if src_k.ndim != 2 or src_k.shape != src_v.shape or src_k.dtype != src_v.dtype:
        raise ValueError("src_k/src_v must be matching [rows, D]")
    D = src_k.shape[1]
    G = rows.shape[0]
    if rows.dtype != torch.int32 or rows.ndim != 2 or rows.stride(1) != 1 or row_counts.shape != (G,) \
            or row_counts.dtype != torch.int32:
        raise ValueError("rows must be [G, stride] int32 with row_counts [G] int32")
    if cur_k.shape != (G, D) or cur_v.shape != (G, D) or cur_k.dtype != src_k.dtype or cur_v.dtype != src_k.dtype:
        raise ValueError("cur_k/cur_v must be [G, D] in the cache dtype")
    if dst_k.ndim != 2 or dst_k.shape != dst_v.shape or dst_k.shape[1] != D or dst_k.dtype != src_k.dtype:
        raise ValueError("dst_k/dst_v must be [capacity, D] in the cache dtype")
    if cu_seqlens.dtype != torch.int32 or cu_seqlens.shape != (G + 1,):
        raise ValueError("cu_seqlens must be [G + 1] int32")
    _require_contiguous(src_k, src_v, cur_k, cur_v, dst_k, dst_v, row_counts, cu_seqlens, what="gather_union")
    dev = _require_device(rows, row_counts, cur_k, cur_v, dst_k, dst_v, cu_seqlens, error_flag,
                          what="gather_union")
    sk, sv = _slab_source(src_k, src_v)
    if resident is not None:
        rm, pk, pv, pcu, st = (resident["map"], resident["prev_k"], resident["prev_v"], resident["prev_cu"],
                               resident.get("stats"))
        if rm.dtype != torch.int64 or rm.ndim != 2 or rm.shape[0] != G or not rm.is_contiguous():
            raise ValueError("the resident map must be contiguous [G, positions] int64")
        if pk.shape != pv.shape or pk.ndim != 2 or pk.shape[1] != D or pk.dtype != src_k.dtype \
                or pcu.dtype != torch.int32 or pcu.shape != (G + 1,) or int(resident["epoch"]) < 1:
            raise ValueError("prev_k/prev_v [capacity, D] and prev_cu [G + 1] int32 must match, epoch >= 1")
        if st is not None and (st.dtype != torch.int64 or st.shape != (2,)):
            raise ValueError("resident stats must be [2] int64")
        _require_contiguous(pk, pv, pcu, what="gather_union")
        _require_device(rm, pk, pv, pcu, st, what="gather_union")
    with on_device(dev):
        if resident is None:
            check(hip().tw_gather_union(sk, sv, src_k.shape[0], entry_row0, entry_row_step, ptr(rows),
                                        rows.stride(0), ptr(row_counts), G, max_count, ptr(cur_k), ptr(cur_v), D,
                                        src_k.element_size(), dst_k.shape[0], ptr(dst_k), ptr(dst_v),
                                        ptr(cu_seqlens), ptr(error_flag), stream_handle(dev)), "gather_union")
        else:
            check(hip().tw_gather_union_resident(
                sk, sv, src_k.shape[0], entry_row0, entry_row_step, ptr(rows), rows.stride(0), ptr(row_counts), G,
                max_count, ptr(cur_k), ptr(cur_v), D, src_k.element_size(), dst_k.shape[0], ptr(dst_k),
                ptr(dst_v), ptr(cu_seqlens), ptr(error_flag), ptr(rm), rm.shape[1], int(resident["epoch"]),
                ptr(pk), ptr(pv), ptr(pcu), pk.shape[0], ptr(st), stream_handle(dev)), "gather_union_resident")


def gather_heads(
    src_k: torch.Tensor,
    src_v: torch.Tensor,
    sel_pages: Optional[torch.Tensor],
    cur_k: torch.Tensor,
    cur_v: torch.Tensor,
    dst_k: torch.Tensor,
    dst_v: torch.Tensor,
    *,
    entry_row0: int,
    entry_row_step: int,
    sink: int,
    recent: int,
    block_size: int,
    length: int,
    num_heads: int,
    dst_strides: tuple[int, int, int],
    error_flag: Optional[torch.Tensor] = None,
) -> None:
    """Per-query-head rows sink ++ own pages ++ recent ++ decode token into
    dst rows g*sg + r*sr + t*st (dst_k/dst_v [capacity, D]).  sel_pages
    [G, R, k] int32 device (None or k = 0: no pages)."""
    if src_k.ndim != 2 or src_k.shape != src_v.shape or src_k.dtype != src_v.dtype:
        raise ValueError("src_k/src_v must be matching [rows, D]")
    D = src_k.shape[1]
    G = cur_k.shape[0]
    R = num_heads
    k = 0 if sel_pages is None else sel_pages.shape[2]
    if sel_pages is not None and (sel_pages.dtype != torch.int32 or sel_pages.shape[:2] != (G, R)
                                  or not sel_pages.is_contiguous()):
        raise ValueError("sel_pages must be contiguous [G, R, k] int32")
    if cur_k.shape != (G, D) or cur_v.shape != (G, D) or cur_k.dtype != src_k.dtype or cur_v.dtype != src_k.dtype:
        raise ValueError("cur_k/cur_v must be [G, D] in the cache dtype")
    if dst_k.ndim != 2 or dst_k.shape != dst_v.shape or dst_k.shape[1] != D or dst_k.dtype != src_k.dtype:
        raise ValueError("dst_k/dst_v must be [capacity, D] in the cache dtype")
    _require_contiguous(src_k, src_v, cur_k, cur_v, dst_k, dst_v, what="gather_heads")
    dev = _require_device(sel_pages, cur_k, cur_v, dst_k, dst_v, error_flag, what="gather_heads")
    sk, sv = _slab_source(src_k, src_v)
    sg, sr, st = dst_strides
    with on_device(dev):
        check(hip().tw_gather_heads(sk, sv, src_k.shape[0], entry_row0, entry_row_step, ptr(sel_pages), G, R, k,
                                    sink, recent, block_size, length, ptr(cur_k), ptr(cur_v), D,
                                    src_k.element_size(), sg, sr, st, dst_k.shape[0], ptr(dst_k), ptr(dst_v),
                                    ptr(error_flag), stream_handle(dev)), "gather_heads")


def append_kv(
    new_k: torch.Tensor,
    new_v: torch.Tensor,
    dst_k: torch.Tensor,
    dst_v: torch.Tensor,
    *,
    first_entry: int,
    position: int,
    device: Optional[torch.device] = None,
) -> None:
    """Write the decode token of n entries into row `position` of
    dst[first_entry + i] (dst: [E, Lmax, D], HBM or pinned host)."""
    if new_k.ndim != 2 or new_k.shape != new_v.shape or new_k.dtype != new_v.dtype:
        raise ValueError("new K/V must be matching [n, D]")
    if dst_k.ndim != 3 or dst_k.shape != dst_v.shape or dst_k.shape[2] != new_k.shape[1] or dst_k.dtype != new_k.dtype:
        raise ValueError("destination must be [E, Lmax, D] matching the new rows")
    _require_contiguous(new_k, new_v, dst_k, dst_v, what="append_kv")
    n, D = new_k.shape
    if first_entry < 0 or first_entry + n > dst_k.shape[0] or not 0 <= position < dst_k.shape[1]:
        raise ValueError("append target outside the cache")
    dev = _require_device(new_k, new_v, what="append_kv")
    if dst_k.is_cuda:
        dk, dv = dst_k.data_ptr(), dst_v.data_ptr()
    else:
        dk, dv = host_device_pointer(dst_k), host_device_pointer(dst_v)
    with on_device(dev):
        check(hip().tw_append_kv(ptr(new_k), ptr(new_v), n, D, new_k.element_size(), dk, dv, dst_k.shape[1],
                                 first_entry, position, stream_handle(dev)), "append_kv")


def host_gather_kv(k: torch.Tensor, v: torch.Tensor, rows: torch.Tensor, out_k: torch.Tensor, out_v: torch.Tensor,
                   threads: Optional[int] = None) -> None:
    """Host (CPU) row gather into staging, e.g. pinned memory for an async
    H2D copy (the reference's CpuKVGather, cpu_kv_gather.py:21-36)."""
    tensors = (k, v, rows, out_k, out_v)
    if any(t.device.type != "cpu" or not t.is_contiguous() for t in tensors):
        raise ValueError("CPU contiguous tensors required")
    if k.ndim != 2 or k.shape != v.shape or k.dtype != v.dtype:
        raise ValueError("invalid source layout")
    if rows.ndim != 1 or rows.dtype != torch.int64:
        raise ValueError("int64 row indices required")
    if out_k.shape != (rows.numel(), k.shape[1]) or out_k.shape != out_v.shape:
        raise ValueError("invalid output layout")
    if out_k.dtype != k.dtype or out_v.dtype != k.dtype:
        raise ValueError("dtype mismatch")
    if rows.numel() == 0:
        return
    rc = _native.host().tw_host_gather_kv(k.data_ptr(), v.data_ptr(), out_k.data_ptr(), out_v.data_ptr(),
                                          rows.data_ptr(), rows.numel(), k.shape[0], k.shape[1] * k.element_size(),
                                          int(threads or torch.get_num_threads()))
    if rc:
        raise ValueError("row index out of bounds")


# ------------------------------------------------- decode-step element-wise
def add_rms_norm(h: torch.Tensor, delta: Optional[torch.Tensor], weight: torch.Tensor, eps: float,
                 out: torch.Tensor) -> torch.Tensor:
    """h += delta (when given), out = weight * rms_norm(h): the decoder layer's
    residual add and LlamaRMSNorm in one launch.  h/delta/out [rows, H]
    contiguous fp16/bf16, weight [H]."""
    if h.dtype not in (torch.float16, torch.bfloat16) or h.ndim != 2 or not h.is_contiguous():
        raise ValueError("h must be contiguous [rows, H] fp16/bf16")
    rows, H = h.shape
    for t in (delta, out):
        if t is not None and (t.shape != h.shape or t.dtype != h.dtype or not t.is_contiguous()):
            raise ValueError("delta/out must match h")
    if weight.shape != (H,) or weight.dtype != h.dtype or not weight.is_contiguous():
        raise ValueError("weight must be [H] in h's dtype")
    dev = _require_device(h, delta, weight, out, what="add_rms_norm")
    with on_device(dev):
        check(hip().tw_add_rms_norm(ptr(h), ptr(delta), ptr(weight), float(eps), ptr(out), rows, H, _dt(h),
                                    stream_handle(dev)), "add_rms_norm")
    return out


def rope_qk(q: torch.Tensor, k: torch.Tensor, cos_table: torch.Tensor, sin_table: torch.Tensor,
            position: torch.Tensor, q32: Optional[torch.Tensor] = None) -> None:
    """apply_rotary_pos_emb of q [Hq, D] and k [Hk, D] in place at the device
    position (int64 [1]) of the cos/sin tables [positions, D]; q32 [Hq, D]
    fp32 receives the rotated q."""
    if q.ndim != 2 or k.ndim != 2 or q.shape[1] != k.shape[1] or q.dtype != k.dtype \
            or q.dtype not in (torch.float16, torch.bfloat16) or not q.is_contiguous() or not k.is_contiguous():
        raise ValueError("q [Hq, D] and k [Hk, D] must be contiguous fp16/bf16")
    D = q.shape[1]
    if cos_table.dtype != q.dtype or sin_table.shape != cos_table.shape or cos_table.ndim != 2 \
            or cos_table.shape[1] != D or not cos_table.is_contiguous() or not sin_table.is_contiguous():
        raise ValueError("cos/sin tables must be contiguous [positions, D] in q's dtype")
    if position.dtype != torch.int64 or position.numel() != 1:
        raise ValueError("position must be one int64")
    if q32 is not None and (q32.dtype != torch.float32 or q32.shape != q.shape or not q32.is_contiguous()):
        raise ValueError("q32 must be contiguous fp32 like q")
    dev = _require_device(q, k, cos_table, sin_table, position, q32, what="rope_qk")
    with on_device(dev):
        check(hip().tw_rope_qk(ptr(q), ptr(k), q.shape[0], k.shape[0], D, ptr(cos_table), ptr(sin_table),
                               ptr(position), ptr(q32), _dt(q), stream_handle(dev)), "rope_qk")


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out = silu(gate_up[..., :I]) * gate_up[..., I:] for one row."""
    if gate_up.dtype not in (torch.float16, torch.bfloat16) or not gate_up.is_contiguous() \
            or gate_up.numel() % 2 or out.dtype != gate_up.dtype or not out.is_contiguous() \
            or out.numel() * 2 != gate_up.numel():
        raise ValueError("gate_up [2I] and out [I] must be contiguous fp16/bf16")
    dev = _require_device(gate_up, out, what="silu_mul")
    with on_device(dev):
        check(hip().tw_silu_mul(ptr(gate_up), ptr(out), out.numel(), _dt(out), stream_handle(dev)), "silu_mul")
    return out


def gemv(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], out: torch.Tensor) -> torch.Tensor:
    """out [1, N] = x [1, K] @ weight [N, K]^T (+ bias): nn.Linear for one
    token, memory-bound (fp32 accumulation)."""
    if weight.ndim != 2 or not weight.is_contiguous() or weight.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("weight must be contiguous [N, K] fp16/bf16")
    N, K = weight.shape
    if x.dtype != weight.dtype or x.numel() != K or not x.is_contiguous():
        raise ValueError("x must be contiguous [K] in the weight's dtype")
    if out.dtype != weight.dtype or out.numel() != N or not out.is_contiguous():
        raise ValueError("out must be contiguous [N] in the weight's dtype")
    if bias is not None and (bias.dtype != weight.dtype or bias.numel() != N or not bias.is_contiguous()):
        raise ValueError("bias must be contiguous [N]")
    dev = _require_device(x, weight, bias, out, what="gemv")
    with on_device(dev):
        check(hip().tw_gemv(ptr(weight), ptr(x), ptr(bias), ptr(out), N, K, _dt(weight), stream_handle(dev)), "gemv")
    return out


def rms_norm_gemv(h: torch.Tensor, delta: Optional[torch.Tensor], norm_weight: torch.Tensor, eps: float,
                  h_out: Optional[torch.Tensor], weight: torch.Tensor, bias: Optional[torch.Tensor],
                  out: torch.Tensor, *, epilogue: str = "plain", rope: Optional[tuple] = None,
                  q32: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One-token nn.Linear whose input is the decoder layer's residual add +
    RMSNorm, in one launch: x = norm_weight * rms_norm(h + delta), h_out =
    h + delta (written when delta is given; a buffer other than h and delta),
    out = x @ weight^T (+ bias).  The same bits as add_rms_norm then gemv.

    epilogue "plain": out [N]; "rope": weight is the concatenated q/k/v
    projection and out [N] gets q and k rotated as rope_qk does, rope =
    (Hq, Hk, cos_table, sin_table, position) and q32 [Hq, D] fp32 (nullable)
    the rotated q; "silu": weight is the concatenated gate/up projection
    [2I, K] and out [I] = silu(gate) * up as silu_mul does."""
    if weight.ndim != 2 or not weight.is_contiguous() or weight.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("weight must be contiguous [N, K] fp16/bf16")
    N, K = weight.shape
    for name, t in (("h", h), ("delta", delta), ("h_out", h_out), ("norm_weight", norm_weight)):
        if t is not None and (t.dtype != weight.dtype or t.numel() != K or not t.is_contiguous()):
            raise ValueError(f"{name} must be contiguous [K] in the weight's dtype")
    if delta is not None and (h_out is None or h_out.data_ptr() in (h.data_ptr(), delta.data_ptr())):
        raise ValueError("h_out must be a buffer other than h and delta")
    if bias is not None and (bias.dtype != weight.dtype or bias.numel() != N or not bias.is_contiguous()):
        raise ValueError("bias must be contiguous [N]")
    n_out = N // 2 if epilogue == "silu" else N
    if out.dtype != weight.dtype or out.numel() != n_out or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [{n_out}] in the weight's dtype")
    dev = _require_device(h, delta, norm_weight, h_out, weight, bias, out, q32, what="rms_norm_gemv")
    args = (ptr(h), ptr(delta), ptr(norm_weight), float(eps), ptr(h_out), ptr(weight), ptr(bias), ptr(out), N, K)
    with on_device(dev):
        if epilogue == "plain":
            check(hip().tw_rms_norm_gemv(*args, _dt(weight), stream_handle(dev)), "rms_norm_gemv")
        elif epilogue == "silu":
            if N % 2:
                raise ValueError("the gate/up weight needs an even row count")
            check(hip().tw_rms_norm_gemv_silu(*args, _dt(weight), stream_handle(dev)), "rms_norm_gemv")
        elif epilogue == "rope":
            if rope is None:
                raise ValueError("the rope epilogue needs rope=(Hq, Hk, cos_table, sin_table, position)")
            Hq, Hk, cos_table, sin_table, position = rope
            D = cos_table.shape[1]
            if N % D or N // D < Hq + Hk:
                raise ValueError("the q/k/v weight rows must hold Hq + Hk (+ Hv) heads of head_dim rows")
            if cos_table.dtype != weight.dtype or sin_table.shape != cos_table.shape or cos_table.ndim != 2 \
                    or not cos_table.is_contiguous() or not sin_table.is_contiguous():
                raise ValueError("cos/sin tables must be contiguous [positions, D] in the weight's dtype")
            if position.dtype != torch.int64 or position.numel() != 1:
                raise ValueError("position must be one int64")
            if q32 is not None and (q32.dtype != torch.float32 or q32.numel() != Hq * D or not q32.is_contiguous()):
                raise ValueError("q32 must be contiguous fp32 [Hq, D]")
            _require_device(cos_table, sin_table, position, what="rms_norm_gemv")
            check(hip().tw_rms_norm_gemv_rope(*args, int(Hq), int(Hk), int(D), ptr(cos_table), ptr(sin_table),
                                              ptr(position), ptr(q32), _dt(weight), stream_handle(dev)),
                  "rms_norm_gemv")
        else:
            raise ValueError(f"unknown epilogue {epilogue!r}")
    return out

