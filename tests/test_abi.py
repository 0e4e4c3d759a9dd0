"""CPU checks of the C ABI boundary: both libraries load without a GPU and
export every function declared in include/*.h; argument validation rejects
bad calls before any launch (no device work happens in these tests)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared(header: Path) -> list[str]:
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(tw_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_hip_library_exports_every_declared_symbol():
    from headinfer import _native

    lib = _native.hip()
    names = _declared(ROOT / "include" / "twilight_hip.h")
    assert "tw_quest_select" in names and "tw_decode_attention" in names
    for name in names:
        assert hasattr(lib, name), name
    assert set(_native._HIP_SIGNATURES) >= set(names)


def test_host_library_exports_every_declared_symbol():
    from headinfer import _native

    lib = _native.host()
    names = _declared(ROOT / "include" / "twilight_host.h")
    assert names == ["tw_host_gather_kv", "tw_host_token_union"]
    for name in names:
        assert hasattr(lib, name), name


def test_status_strings_and_version():
    from headinfer import _native

    lib = _native.hip()
    for code in range(6):
        assert lib.tw_status_string(code)
    assert lib.tw_version() >= 1


def test_invalid_arguments_rejected_without_launch():
    from headinfer import _native

    lib = _native.hip()
    # null pointers / bad sizes return TW_EINVAL before touching the device
    assert lib.tw_quest_score(None, None, None, 0, 1, 1, 1, 128, 128, None, None) == _native.TW_EINVAL
    assert lib.tw_topk_sorted(None, 1, 10, 10, 3, None, None, 0, None) == _native.TW_EINVAL
    assert lib.tw_topk_sorted_workspace_size(4, 8192) == 0 and lib.tw_topk_sorted_workspace_size(4, 8193) > 0
    assert lib.tw_twilight_max_candidates() == 16384
    assert lib.tw_build_page_metadata(None, 0, 1, 16, 3, 0, 0, 16, None, None, 0, None, None, None, 0,
                                      None) == _native.TW_EINVAL
    assert lib.tw_decode_attention(None, None, None, 0, 1, 1, 128, None, None, None, 0, 0, None, 1, -1, 0, None,
                                   None, 1.0, None, None, 0, None) == _native.TW_EINVAL
    assert lib.tw_append_kv(None, None, 1, 128, 2, None, None, 10, 0, 10, None) == _native.TW_EINVAL
    with pytest.raises(ValueError):
        _native.check(_native.TW_EINVAL, "probe")
    with pytest.raises(RuntimeError):
        _native.check(_native.TW_ENOMEM, "probe")


def test_host_gather_matches_reference_native_and_index_select():
    """The host gather native against index_select and, when built, the
    reference's own cpu_kv_run_gather.so (oracle/_ref)."""
    import torch

    from headinfer import kernels

    g = torch.Generator().manual_seed(1234)
    k = torch.randn((10000, 128), generator=g).to(torch.bfloat16)
    v = torch.randn_like(k.float()).to(torch.bfloat16)
    patterns = [
        torch.empty(0, dtype=torch.long), torch.tensor([9999]), torch.arange(9999),
        torch.randint(10000, (8192,), generator=g), torch.arange(8192).flip(0),
        torch.cat([torch.arange(100, 500), torch.tensor([0, 0, 9999]), torch.arange(1000, 7000)]),
        torch.cat([torch.arange(i, i + n) for i, n in ((100, 15), (300, 16), (600, 17), (1000, 33))]),
    ]
    ref_lib = ROOT / "oracle" / "_ref" / "cpu_kv_run_gather.so"
    ref = ctypes.CDLL(str(ref_lib)) if ref_lib.exists() else None
    for threads in (1, 2, 6):
        for rows in patterns:
            a = torch.full((rows.numel() + 2, 128), -42.0, dtype=k.dtype)
            b = torch.full_like(a, -42.0)
            kernels.host_gather_kv(k, v, rows, a[1:-1], b[1:-1], threads=threads)
            assert torch.equal(a[1:-1], k.index_select(0, rows)) and torch.equal(b[1:-1], v.index_select(0, rows))
            assert (a[[0, -1]] == -42).all() and (b[[0, -1]] == -42).all()
            if ref is not None and rows.numel():
                ra = torch.empty((rows.numel(), 128), dtype=k.dtype)
                rb = torch.empty_like(ra)
                rc = ref.gather_kv(ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(v.data_ptr()),
                                   ctypes.c_void_p(ra.data_ptr()), ctypes.c_void_p(rb.data_ptr()),
                                   ctypes.c_void_p(rows.data_ptr()), ctypes.c_int64(rows.numel()),
                                   ctypes.c_int64(10000), ctypes.c_int64(256), ctypes.c_int(threads))
                assert rc == 0
                assert torch.equal(ra, a[1:-1]) and torch.equal(rb, b[1:-1])
    for bad in (-1, 10000):
        with pytest.raises(ValueError):
            kernels.host_gather_kv(k, v, torch.tensor([bad]), a[:1], b[:1])
