"""CPU oracle (test infrastructure only; never imported by the product).

ctypes wrappers over ``twilight_oracle.c`` and numpy references.  Arrays of
16-bit keys are passed as their raw ``uint16`` bit patterns; ``dtype`` is one
of ``"f16"``, ``"bf16"``, ``"f32"``.
"""

from __future__ import annotations

import ctypes
import math
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle.so"
_DT = {"f16": 0, "bf16": 1, "f32": 2}
_lib = None

__all__ = [
    "lib",
    "DTYPES",
    "f16_bits_to_f32",
    "f32_to_f16_bits",
    "bf16_bits_to_f32",
    "f32_to_bf16_bits",
    "to_f32",
    "from_f32",
    "build_page_metadata",
    "int4_dequantize",
    "qfix",
    "quest_score",
    "topk_sorted",
    "quest_row_plan",
    "selection_window",
    "quest_budget",
    "decode_attention",
    "host_gather",
    "det_exp",
    "int4_qk",
    "top_p_count",
    "top_p_threshold",
    "mass",
    "matched_budget_counts",
    "twilight_layer",
]

DTYPES = ("f16", "bf16", "f32")


def lib() -> ctypes.CDLL:
    """Load (building on first use) the oracle's C library."""
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            subprocess.run(["make", "-s", "-C", str(_HERE), "_build/liboracle.so"], check=True)
        L = ctypes.CDLL(str(_LIB_PATH))
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_bf16_to_f32.restype = ctypes.c_float
        L.or_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f32_to_bf16.restype = ctypes.c_uint16
        L.or_f32_to_bf16.argtypes = [ctypes.c_float]
        L.or_build_page_metadata.restype = i32
        L.or_build_page_metadata.argtypes = [vp, i32, i32, i32, i32, i32, vp, vp, vp, vp, vp]
        L.or_int4_dequantize.restype = None
        L.or_int4_dequantize.argtypes = [vp, vp, vp, i32, i64, i32, vp]
        L.or_quest_score.restype = None
        L.or_quest_score.argtypes = [vp, vp, vp, i32, i32, i32, i32, i32, i64, vp]
        L.or_topk_sorted.restype = None
        L.or_topk_sorted.argtypes = [vp, i32, i32, i64, i32, vp]
        L.or_quest_row_plan.restype = i32
        L.or_quest_row_plan.argtypes = [vp, i32, i32, i32, i32, i32, i32, i32, i32, vp, vp]
        L.or_det_exp.restype = ctypes.c_float
        L.or_det_exp.argtypes = [ctypes.c_float]
        L.or_qfix.restype = i32
        L.or_qfix.argtypes = [vp, i32, vp, vp, vp]
        L.or_int4_qk.restype = None
        L.or_int4_qk.argtypes = [vp, i32, vp, vp, vp, i32, vp, i32, ctypes.c_float, vp]
        L.or_top_p_count.restype = i32
        L.or_top_p_count.argtypes = [vp, i32, ctypes.c_float, vp]
        L.or_top_p_threshold.restype = ctypes.c_uint64
        L.or_top_p_threshold.argtypes = [ctypes.c_uint64, ctypes.c_float]
        L.or_mass.restype = ctypes.c_uint64
        L.or_mass.argtypes = [ctypes.c_float, ctypes.c_float]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


# ------------------------------------------------------------------ dtypes
def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even (NaN -> quiet NaN with the sign kept)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) & 0x8000) | 0x7FC0, r)
    return r.astype(np.uint16)


def to_f32(a: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f32":
        return np.asarray(a, dtype=np.float32)
    return f16_bits_to_f32(a) if dtype == "f16" else bf16_bits_to_f32(a)


def from_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f32":
        return np.asarray(x, dtype=np.float32)
    return f32_to_f16_bits(x) if dtype == "f16" else f32_to_bf16_bits(x)


def _storage(dtype: str):
    return np.float32 if dtype == "f32" else np.uint16


# ------------------------------------------------------------ metadata
def build_page_metadata(keys: np.ndarray, dtype: str, sink: int, block_size: int, *, pages=True, quant=True):
    """Page min/max (quest_offload_cache.py:276-289) and INT4 pack
    (twilight_offload_cache.py:25-37) of one entry's keys [T, D].

    Returns (page_min, page_max, packed, scale, minimum); disabled parts are
    None."""
    keys = np.ascontiguousarray(keys, dtype=_storage(dtype))
    T, D = keys.shape
    P = (T - sink) // block_size if T > sink else 0
    st = _storage(dtype)
    pmin = np.zeros((P, D), st) if pages else None
    pmax = np.zeros((P, D), st) if pages else None
    packed = np.zeros((T, D // 2), np.uint8) if quant else None
    scale = np.zeros(T, st) if quant else None
    minimum = np.zeros(T, st) if quant else None

    def p(a):
        return None if a is None else _ptr(a)

    rc = lib().or_build_page_metadata(_ptr(keys), T, D, _DT[dtype], sink, block_size, p(pmin), p(pmax), p(packed),
                                      p(scale), p(minimum))
    if rc:
        raise ValueError("invalid metadata arguments")
    return pmin, pmax, packed, scale, minimum


def int4_dequantize(packed: np.ndarray, scale: np.ndarray, minimum: np.ndarray, dtype: str) -> np.ndarray:
    """affine_int4_dequantize (twilight_offload_cache.py:40-47)."""
    packed = np.ascontiguousarray(packed, np.uint8)
    N, half = packed.shape
    out = np.zeros((N, 2 * half), np.float32)
    lib().or_int4_dequantize(_ptr(packed), _ptr(np.ascontiguousarray(scale, _storage(dtype))),
                             _ptr(np.ascontiguousarray(minimum, _storage(dtype))), _DT[dtype], N, 2 * half,
                             _ptr(out))
    return out


# ------------------------------------------------------------- Quest
def quest_score(q: np.ndarray, page_min: np.ndarray, page_max: np.ndarray, dtype: str) -> np.ndarray:
    """fused_quest_score order (twilight_fused_quest.py:12-32).

    q [G, R, D] fp32; page_min/page_max [G, P, D] -> [G, R, P] fp32."""
    q = np.ascontiguousarray(q, np.float32)
    G, R, D = q.shape
    pmin = np.ascontiguousarray(page_min, _storage(dtype))
    pmax = np.ascontiguousarray(page_max, _storage(dtype))
    P = pmin.shape[1]
    out = np.zeros((G, R, P), np.float32)
    lib().or_quest_score(_ptr(q), _ptr(pmin), _ptr(pmax), _DT[dtype], G, R, P, D, P * D, _ptr(out))
    return out


def topk_sorted(scores: np.ndarray, k: int) -> np.ndarray:
    """topk(sorted=False).indices.sort() with ties to the lowest index
    (quest_offload_cache.py:373-374)."""
    s = np.ascontiguousarray(scores, np.float32)
    lead = s.shape[:-1]
    P = s.shape[-1]
    flat = s.reshape(-1, P)
    out = np.zeros((flat.shape[0], k), np.int64)
    lib().or_topk_sorted(_ptr(flat), flat.shape[0], P, P, k, _ptr(out))
    return out.reshape(*lead, k)


def quest_row_plan(sel: np.ndarray, P: int, sink: int, recent: int, block_size: int, length: int,
                   append_position: int = -1):
    """Row plan of one KV group: sink ++ union pages ++ recent (++ append)."""
    sel = np.ascontiguousarray(sel, np.int64)
    R, k = sel.shape
    cap = length + 1
    rows = np.zeros(cap, np.int32)
    masks = np.zeros(cap, np.uint8)
    n = lib().or_quest_row_plan(_ptr(sel), R, k, P, sink, recent, block_size, length, append_position, _ptr(rows),
                                _ptr(masks))
    return rows[:n].copy(), masks[:n].copy()


def selection_window(length: int, sink: int, recent: int):
    """(sink_end, recent_start, eligible) of quest_offload_cache.py:330-333."""
    sink_end = min(sink, length)
    recent_start = max(sink_end, length - max(0, recent - 1))
    return sink_end, recent_start, max(0, recent_start - sink_end)


def quest_budget(length: int, sink: int, recent: int, block_size: int, fraction: float, meta_pages: int):
    """(candidate_pages, budget) of quest_offload_cache.py:333-346."""
    _, _, eligible = selection_window(length, sink, recent)
    cand = eligible // block_size
    budget = min(cand, max(1, math.ceil(fraction * eligible / block_size)))
    cand = min(cand, meta_pages)
    return cand, min(budget, cand)


# ------------------------------------------------------------ attention
def decode_attention(q: np.ndarray, keys: np.ndarray, values: np.ndarray, scale: float,
                     masks: np.ndarray | None = None) -> np.ndarray:
    """float64 softmax(q k^T * scale) v for one group: q [R, D], keys/values
    [N, D] (float arrays), masks [N] head bitmask or None.  The SDPA math
    reference of decode_reference_attention.py:18-69 at q_len 1."""
    q = np.asarray(q, np.float64)
    k = np.asarray(keys, np.float64)
    v = np.asarray(values, np.float64)
    R = q.shape[0]
    out = np.zeros((R, v.shape[1]), np.float64)
    for r in range(R):
        s = (k @ q[r]) * scale
        if masks is not None:
            vis = ((masks.astype(np.int64) >> r) & 1).astype(bool)
            s = np.where(vis, s, -np.inf)
        m = s.max()
        p = np.exp(s - m)
        out[r] = (p @ v) / p.sum()
    return out


def host_gather(src: np.ndarray, rows: np.ndarray) -> np.ndarray:
    """index_select of rows (quest_offload_cache.py:580-587)."""
    return src[np.asarray(rows, np.int64)]


# ------------------------------------------------------------- Twilight
def det_exp(x: float) -> float:
    """The shared deterministic exp of x <= 0 (twilight_oracle.c)."""
    return float(lib().or_det_exp(float(np.float32(x))))


def qfix(q: np.ndarray) -> tuple[np.ndarray, int, int, bool]:
    """Fixed-point form of a query head: (Q [D] int32, sum Q, shift, finite)
    with q~ = Q * 2^shift (see or_qfix)."""
    q = np.ascontiguousarray(q, np.float32)
    Q = np.zeros(q.shape[0], np.int32)
    qs = ctypes.c_int32()
    ok = ctypes.c_int()
    shift = lib().or_qfix(_ptr(q), q.shape[0], _ptr(Q), ctypes.byref(qs), ctypes.byref(ok))
    return Q, int(qs.value), int(shift), bool(ok.value)


def int4_qk(q: np.ndarray, packed: np.ndarray, scale: np.ndarray, minimum: np.ndarray, dtype: str,
            rows: np.ndarray, qk_scale: float) -> np.ndarray:
    """INT4 QK estimate of one query head q [D] over candidate rows: the
    exact integer dot of the codes with q's fixed-point form, then
    qk_scale * (scale * dot + min * sum q~) in fp32 (see or_int4_qk)."""
    q = np.ascontiguousarray(q, np.float32)
    packed = np.ascontiguousarray(packed, np.uint8)
    rows = np.ascontiguousarray(rows, np.int64)
    out = np.zeros(rows.shape[0], np.float32)
    lib().or_int4_qk(_ptr(q), q.shape[0], _ptr(packed), _ptr(np.ascontiguousarray(scale, _storage(dtype))),
                     _ptr(np.ascontiguousarray(minimum, _storage(dtype))), _DT[dtype], _ptr(rows), rows.shape[0],
                     float(np.float32(qk_scale)), _ptr(out))
    return out


def top_p_count(logits: np.ndarray, top_p: float) -> tuple[int, int]:
    """(desired, Z) of the exact top-p count."""
    lg = np.ascontiguousarray(logits, np.float32)
    z = ctypes.c_uint64()
    d = lib().or_top_p_count(_ptr(lg), lg.shape[0], float(np.float32(top_p)), ctypes.byref(z))
    return int(d), int(z.value)


def top_p_threshold(z: int, top_p: float) -> int:
    return int(lib().or_top_p_threshold(z, float(np.float32(top_p))))


def mass(logit: float, lmax: float) -> int:
    return int(lib().or_mass(float(np.float32(logit)), float(np.float32(lmax))))


def matched_budget_counts(desired, target_total, capacities):
    """Largest-remainder reallocation (twilight_offload_cache.py:50-86),
    restated: each head keeps at least 1; the remaining target is split in
    proportion to desired (float64), floors first, then +1 by (fractional
    remainder desc, desired desc, index asc) until the target is met; any
    excess is taken back from the heads with the smallest (desired, index)."""
    n = len(desired)
    if n == 0 or n != len(capacities):
        raise ValueError("desired and capacities must be non-empty and aligned")
    if min(desired) <= 0 or min(capacities) <= 0:
        raise ValueError("desired counts and capacities must be positive")
    if target_total < n or target_total > sum(capacities):
        raise ValueError("target_total is infeasible")
    remaining = target_total - n
    total = float(sum(float(v) for v in desired))
    raw = [remaining * float(v) / total for v in desired]
    counts = [1 + min(capacities[i] - 1, math.floor(raw[i])) for i in range(n)]
    while sum(counts) < target_total:
        order = sorted((i for i in range(n) if counts[i] < capacities[i]),
                       key=lambda i: (-(raw[i] - math.floor(raw[i])), -desired[i], i))
        best = order[0]
        counts[best] += 1
        raw[best] = math.floor(raw[best])
    while sum(counts) > target_total:
        worst = min((i for i in range(n) if counts[i] > 1), key=lambda i: (desired[i], i))
        counts[worst] -= 1
    return counts


def twilight_layer(q: np.ndarray, page_min: np.ndarray, page_max: np.ndarray, packed: np.ndarray,
                   scale: np.ndarray, minimum: np.ndarray, dtype: str, *, length: int, sink: int, recent: int,
                   block_size: int, b0_pages: int, top_p: float, budget_mode: str = "dynamic",
                   fixed_pages: int = 0, qk_scale: float | None = None, target_total: int | None = None):
    """Twilight selection of one KV group (prepare_layer_selection,
    twilight_offload_cache.py:996-1614) in the orders twilight_oracle.c defines.

    q [R, D] fp32; page_min/page_max [P, D] (the P scored pages); packed
    [T, D/2], scale/minimum [T] (storage of dtype).  Returns a dict with the
    stage-1 pages [R, b0] (ascending), logits [R, N], desired [R], allocated
    [R], selected positions per head (ascending) and the GQA union rows."""
    R, D = q.shape
    P = page_min.shape[0]
    qk_scale = float(np.float32(1.0 / math.sqrt(D))) if qk_scale is None else qk_scale
    sink_end, recent_start, _ = selection_window(length, sink, recent)
    sc = quest_score(q[None], page_min[None], page_max[None], dtype)[0]
    pages = topk_sorted(sc, b0_pages)  # [R, b0] ascending (candidate order)
    offs = np.arange(block_size)
    cand = (sink + pages[:, :, None] * block_size + offs).reshape(R, -1)  # [R, N]
    logits = np.stack([int4_qk(q[r], packed, scale, minimum, dtype, cand[r], qk_scale) for r in range(R)])
    N = cand.shape[1]
    desired = np.array([top_p_count(logits[r], top_p)[0] for r in range(R)])
    if budget_mode == "dynamic":
        allocated = desired.copy()
    else:
        # the cache's target (fixed pages x page size x R) unless one is given
        target = fixed_pages * block_size * R if target_total is None else int(target_total)
        allocated = np.array(matched_budget_counts(list(map(int, desired)), target, [N] * R))
    selected = []
    for r in range(R):
        idx = topk_sorted(logits[r][None], int(allocated[r]))[0]
        selected.append(np.sort(cand[r][idx]))
    union = np.unique(np.concatenate([np.arange(sink_end), *selected, np.arange(recent_start, length)]))
    return {"pages": pages, "candidates": cand, "logits": logits, "desired": desired, "allocated": allocated,
            "selected": selected, "union": union}
