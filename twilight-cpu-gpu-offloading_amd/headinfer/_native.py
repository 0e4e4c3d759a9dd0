"""ctypes bindings of the package's native libraries.

``libtwilight_hip.so`` (gfx950 HIP kernels) and ``libtwilight_host.so`` (host
natives) are loaded the way the reference loads its natives: ``ctypes.CDLL``
with explicit argtypes, raw pointers and an int status
(cpu_kv_gather.py:17-18, resident_zero_copy.py:41-42).  Unlike the reference
nothing is compiled at import time: the libraries are built in-tree ahead of
time (``build_native.py``).  A missing library is an error, never a fallback.

torch is imported first on purpose: the HIP runtime torch ships has the same
soname as /opt/rocm's, so the kernels run on torch's runtime and can take
torch's stream handles directly.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_DIR = Path(__file__).resolve().parent / "_lib"
HIP_LIB = LIB_DIR / "libtwilight_hip.so"
HOST_LIB = LIB_DIR / "libtwilight_host.so"

TW_OK, TW_EINVAL, TW_ERANGE, TW_ENOMEM, TW_EHIP, TW_EUNSUPPORTED = range(6)
DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}

_hip = None
_host = None

vp = ctypes.c_void_p
i32 = ctypes.c_int
i64 = ctypes.c_int64
f32 = ctypes.c_float
f64 = ctypes.c_double
szt = ctypes.c_size_t

_HIP_SIGNATURES = {
    "tw_status_string": (ctypes.c_char_p, [i32]),
    "tw_last_hip_error": (i32, []),
    "tw_version": (i32, []),
    "tw_build_page_metadata": (i32, [vp, i64, i32, i32, i32, i32, i32, i32, vp, vp, i64, vp, vp, vp, i64, vp]),
    "tw_update_page_metadata": (i32, [vp, i64, i32, i32, i32, i32, i32, i32, vp, vp, i64, vp, vp, vp, i64, vp]),
    "tw_update_page_metadata_ragged": (i32, [vp, i64, i32, vp, i32, i32, i32, i32, i32, vp, vp, i32, i64, vp, vp,
                                             vp, i64, vp]),
    "tw_quest_select_ragged": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, i64, vp, i32, vp, vp, vp, vp, i64, i32, i32,
                                     i32, vp, szt, vp]),
    "tw_quest_select_bits": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, i64, vp, i32, vp, vp, vp, i64, i32, i32, i32,
                                   vp, szt, vp]),
    "tw_decode_attention_pages_bits": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, i64, i32, i32, i64, i32, i32, i32,
                                             vp, i32, i32, vp, vp, f32, vp, vp, i64, i32, vp, vp, szt, i32, vp]),
    "tw_decode_attention_pages_ragged": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, i64, i32, i64, i32, i32,
                                               i32, vp, i32, vp, vp, f32, vp, vp, i64, i32, vp, vp, szt, vp]),
    "tw_decode_attention_pages_resident": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, i64, i32, i64, i32,
                                                 i32, i32, vp, i32, i32, vp, vp, f32, vp, vp, vp, i32, i32, vp, vp,
                                                 vp, vp, i32, vp, vp, i64, i32, vp, vp, szt, vp]),
    "tw_add_rms_norm": (i32, [vp, vp, vp, f32, vp, i32, i32, i32, vp]),
    "tw_rope_qk": (i32, [vp, vp, i32, i32, i32, vp, vp, vp, vp, i32, vp]),
    "tw_silu_mul": (i32, [vp, vp, i32, i32, vp]),
    "tw_gemv": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "tw_rms_norm_gemv": (i32, [vp, vp, vp, f32, vp, vp, vp, vp, i32, i32, i32, vp]),
    "tw_rms_norm_gemv_rope": (i32, [vp, vp, vp, f32, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp, vp, vp, vp, i32,
                                    vp]),
    "tw_rms_norm_gemv_silu": (i32, [vp, vp, vp, f32, vp, vp, vp, vp, i32, i32, i32, vp]),
    "tw_int4_dequantize": (i32, [vp, vp, vp, i32, i64, i32, vp, vp]),
    "tw_quest_score": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, i64, vp, vp]),
    "tw_topk_sorted_workspace_size": (szt, [i32, i32]),
    "tw_topk_sorted": (i32, [vp, i32, i32, i64, i32, vp, vp, szt, vp]),
    "tw_quest_select_workspace_size": (szt, [i32, i32, i32]),
    "tw_quest_select": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, i64, i32, vp, vp, vp, vp, vp, i64, vp, vp, vp, i64,
                              i32, i32, i32, i32, i32, vp, szt, vp]),
    "tw_quest_select_static_capacity": (szt, []),
    "tw_quest_select_static": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, i64, i32, vp, vp, vp, vp, vp, i64, vp, vp,
                                     vp, i64, i32, i32, i32, i32, i32, vp]),
    "tw_decode_attention_workspace_size": (szt, [i32, i32, i32, i32]),
    "tw_decode_attention": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, i64, i64, vp, i32, i32, i32, vp, vp,
                                  f32, vp, vp, szt, vp]),
    "tw_decode_attention_rows_append": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, i64, i64, i32, vp, vp,
                                              i64, vp, f32, i32, vp, vp, i64, i32, vp, vp, vp, i64, vp, vp, szt,
                                              vp]),
    "tw_decode_attention_pages": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, i64, i32, i64, i32, i32, i32, i32,
                                        i32, vp, vp, f32, vp, vp, szt, vp]),
    "tw_twilight_qk": (i32, [vp, i32, i32, i32, vp, vp, vp, i32, i64, i64, vp, vp, vp, i64, i32, i32, i32, f32, vp, vp,
                             vp, vp]),
    "tw_twilight_select_pages": (i32, [vp, i32, i32, i32, vp, i32, f32, vp, vp, i64, vp, i32, i32, i32, i32, vp, i32,
                                       vp, szt, vp]),
    "tw_decode_attention_page_rows": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, i64, i32, i64, i32, i32, i32,
                                            vp, i32, i32, vp, vp, f32, vp, vp, i64, i32, vp, vp, vp, i64, vp, vp, szt,
                                            vp]),
    "tw_twilight_union_record_words": (i32, [i32]),
    "tw_twilight_select_fused_workspace_size": (szt, [i32, i32, i32, i32]),
    "tw_twilight_select_fused": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, i64, vp, vp, vp, i64, i64, i32, f32, f32,
                                       i32, i32, i32, vp, i32, vp, vp, vp, vp, i64, vp, szt, vp]),
    "tw_twilight_select_fused_phase": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, i64, vp, vp, vp, i64, i64, i32, f32,
                                             f32, i32, i32, i32, vp, i32, vp, vp, vp, vp, i64, vp, szt, i32, vp]),
    "tw_twilight_select_fused_matched": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, i64, vp, vp, vp, i64, i64, i32,
                                               f32, f32, i32, i32, i32, vp, i32, i32, f64, vp, vp, vp, vp, vp, i64,
                                               vp, szt, vp]),
    "tw_twilight_select_fused_matched_part": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, i64, vp, vp, vp, i64, i64,
                                                    i32, f32, f32, i32, i32, i32, vp, i32, i32, f64, vp, vp, vp, vp,
                                                    vp, i64, i32, vp, i32, i32, vp, szt, vp]),
    "tw_decode_attention_union": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, i64, i32, i32, i64, i32, i32, i32, vp,
                                        i32, i32, vp, vp, f32, vp, vp, i64, i32, vp, vp, vp, i64, vp, vp, szt, i32,
                                        vp]),
    "tw_decode_attention_union_resident": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, i64, i32, i32, i64, i32, i32,
                                                 i32, vp, i32, i32, vp, vp, f32, vp, vp, vp, i32, i32, vp, vp, vp,
                                                 vp, i32, vp, vp, i64, i32, vp, vp, vp, i64, vp, vp, szt, i32,
                                                 vp]),
    "tw_int4_qk_positions": (i32, [vp, i32, i32, i32, vp, vp, vp, i32, i64, i64, vp, i32, f32, i32, vp, vp]),
    "tw_twilight_select_workspace_size": (szt, [i32, i32, i32]),
    "tw_twilight_max_candidates": (i32, []),
    "tw_twilight_select": (i32, [vp, i32, i32, i32, vp, i32, f32, i32, i32, vp, vp, vp, vp, vp, i64, i32, i32, i32,
                                 i32, i32, vp, szt, vp]),
    "tw_twilight_select_ragged": (i32, [vp, i32, i32, i32, vp, i32, f32, vp, vp, vp, vp, vp, i64, i32, i32, i32, vp,
                                        i32, i32, vp, szt, vp]),
    "tw_decode_attention_pages_phase": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, i64, i32, i64, i32, i32,
                                              i32, i32, i32, vp, vp, f32, vp, vp, szt, i32, vp]),
    "tw_gather_rows": (i32, [vp, vp, i64, vp, vp, i64, i64, i32, i32, vp, vp, vp, vp]),
    "tw_gather_union": (i32, [vp, vp, i64, i64, i64, vp, i64, vp, i32, i32, vp, vp, i32, i32, i64, vp, vp, vp, vp,
                              vp]),
    "tw_gather_union_resident": (i32, [vp, vp, i64, i64, i64, vp, i64, vp, i32, i32, vp, vp, i32, i32, i64, vp, vp,
                                       vp, vp, vp, i64, i32, vp, vp, vp, i64, vp, vp]),
    "tw_gather_heads": (i32, [vp, vp, i64, i64, i64, vp, i32, i32, i32, i32, i32, i32, i32, vp, vp, i32, i32, i64,
                              i64, i64, i64, vp, vp, vp, vp]),
    "tw_host_device_pointer": (i32, [vp, ctypes.POINTER(ctypes.c_void_p)]),
    "tw_append_kv": (i32, [vp, vp, i32, i32, i32, vp, vp, i64, i32, i64, vp]),
}

_HOST_SIGNATURES = {
    "tw_host_gather_kv": (i32, [vp, vp, vp, vp, vp, i64, i64, i64, i32]),
    "tw_host_token_union": (i64, [ctypes.POINTER(ctypes.c_void_p), vp, i32, i64, vp, vp]),
}


def _load(path: Path, signatures: dict) -> ctypes.CDLL:
    if not path.exists():
        raise RuntimeError(
            f"{path.name} is not built; run `python build_native.py` in {path.parent.parent.parent} "
            "(or __graft_entry__.build()) first"
        )
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in signatures.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def hip() -> ctypes.CDLL:
    """The gfx950 kernel library (loaded once)."""
    global _hip
    if _hip is None:
        _hip = _load(HIP_LIB, _HIP_SIGNATURES)
    return _hip


def host() -> ctypes.CDLL:
    """The host natives library (loaded once)."""
    global _host
    if _host is None:
        _host = _load(HOST_LIB, _HOST_SIGNATURES)
    return _host


def check(status: int, what: str) -> None:
    """Map a C ABI status to the reference's exception types."""
    if status == TW_OK:
        return
    text = hip().tw_status_string(status).decode()
    if status in (TW_EINVAL, TW_ERANGE):
        raise ValueError(f"{what}: {text}")
    if status == TW_EHIP:
        raise RuntimeError(f"{what}: {text} (hipError {hip().tw_last_hip_error()})")
    raise RuntimeError(f"{what}: {text}")


def stream_handle(device: torch.device | None = None) -> int:
    """The hipStream_t of torch's current stream on ``device``."""
    index = torch.cuda.current_device() if device is None or device.index is None else device.index
    return _raw_stream(index)


def _raw_stream_of(index: int) -> int:
    return torch.cuda.current_stream(index).cuda_stream


# torch's current raw stream without building a Stream object (a few
# microseconds a call on the eager decode path)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None) or _raw_stream_of


class _NoGuard:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NO_GUARD = _NoGuard()


def on_device(device: torch.device):
    """torch.cuda.device(device), or nothing to do when it is already current."""
    if device.index is None or device.index == torch.cuda.current_device():
        return _NO_GUARD
    return torch.cuda.device(device)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
