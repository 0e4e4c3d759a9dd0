"""The reference's host-native helper modules on this package's natives.

The cases are those of the reference's own tests: scripts/test_cpu_kv_gather_v1.py:7-22
(empty / singleton / 8192 random rows, invalid indices) and
scripts/test_cpu_kv_run_gather_v1.py:6-30 (run patterns, 1/2/6 threads, guard rows
around the output slice), with index_select as the oracle; the token union is
checked against np.unique (the set identity of scripts/test_twilight_offload_cache_v1.py
:291-294).  The reference pins its staging rows; pinning needs a device and does
not change a CPU copy, so these use pageable rows.  CPU only."""

from __future__ import annotations

import numpy as np
import pytest
import torch


def test_cpu_kv_gather_reference_cases():
    from headinfer.cpu_kv_gather import CpuKVGather

    gather = CpuKVGather()
    g = torch.Generator().manual_seed(123)
    for n in (0, 1, 8192):
        k = torch.randn((10000, 128), generator=g).to(torch.bfloat16)
        v = torch.randn((10000, 128), generator=g).to(torch.bfloat16)
        rows = torch.randint(10000, (n,), generator=g)
        a = torch.empty(n, 128, dtype=k.dtype)
        b = torch.empty_like(a)
        gather(k, v, rows, a, b)
        assert torch.equal(a, k[rows]) and torch.equal(b, v[rows])
    for bad in (-1, 10000):
        with pytest.raises(ValueError):
            gather(k, v, torch.tensor([bad]), a[:1], b[:1])


def test_cpu_kv_gather_rejects_bad_layouts():
    from headinfer.cpu_kv_gather import CpuKVGather

    gather = CpuKVGather()
    k = torch.zeros(16, 8, dtype=torch.float16)
    v = torch.zeros_like(k)
    rows = torch.arange(4)
    out = torch.empty(4, 8, dtype=k.dtype)
    with pytest.raises(ValueError, match="int64"):
        gather(k, v, rows.to(torch.int32), out, out.clone())
    with pytest.raises(ValueError, match="source layout"):
        gather(k, v[:, :4].contiguous(), rows, out, out.clone())
    with pytest.raises(ValueError, match="output layout"):
        gather(k, v, rows, out[:3], out.clone())
    with pytest.raises(ValueError, match="dtype"):
        gather(k, v, rows, out.float(), out.float())
    with pytest.raises(ValueError, match="contiguous"):
        gather(k.t(), v.t(), rows, out, out.clone())


def test_cpu_kv_run_gather_reference_cases():
    from headinfer.cpu_kv_run_gather import CpuKVRunGather

    gather = CpuKVRunGather()
    g = torch.Generator().manual_seed(1234)
    k = torch.randn((10000, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((10000, 128), generator=g).to(torch.bfloat16)
    patterns = [
        torch.empty(0, dtype=torch.long), torch.tensor([9999]), torch.arange(9999),
        torch.randint(10000, (8192,), generator=g), torch.arange(8192).flip(0),
        torch.cat([torch.arange(100, 500), torch.tensor([0, 0, 9999]), torch.arange(1000, 7000)]),
        torch.cat([torch.arange(i, i + n) for i, n in ((100, 15), (300, 16), (600, 17), (1000, 33))]),
    ]
    threads0 = torch.get_num_threads()
    cases = 0
    try:
        for threads in (1, 2, 6):
            torch.set_num_threads(threads)
            for rows in patterns:
                a = torch.full((rows.numel() + 2, 128), -42.0, dtype=k.dtype)
                b = torch.full_like(a, -42.0)
                gather(k, v, rows, a[1:-1], b[1:-1])
                assert torch.equal(a[1:-1], k.index_select(0, rows))
                assert torch.equal(b[1:-1], v.index_select(0, rows))
                assert (a[[0, -1]] == -42).all() and (b[[0, -1]] == -42).all()
                cases += 1
    finally:
        torch.set_num_threads(threads0)
    assert cases == 21
    for bad in (-1, 10000):
        with pytest.raises(ValueError):
            gather(k, v, torch.tensor([bad]), a[:1], b[:1])


def test_cpu_token_union_matches_unique_and_rejects_outside():
    from headinfer.cpu_token_union import CpuTokenUnion

    rng = np.random.default_rng(7)
    union = CpuTokenUnion(5000)
    for length in (0, 1, 17, 4096, 5000):
        lists = [torch.from_numpy(rng.integers(0, max(length, 1), size=int(rng.integers(0, 600)))).to(torch.int64)
                 for _ in range(4)] if length else [torch.empty(0, dtype=torch.int64)]
        lists.append(torch.empty(0, dtype=torch.int64))
        got = union(lists, length)
        want = np.unique(np.concatenate([t.numpy() for t in lists])) if length else np.empty(0, np.int64)
        assert got.dtype == torch.int64 and np.array_equal(got.numpy(), want)
    first = union([torch.tensor([3, 1])], 10)
    union([torch.tensor([7])], 10)
    assert first.tolist() == [1, 3]          # results own their memory
    with pytest.raises(ValueError, match="outside history"):
        union([torch.tensor([10])], 10)
    with pytest.raises(ValueError, match="outside history"):
        union([torch.tensor([-1])], 10)
    with pytest.raises(ValueError, match="invalid union length"):
        union([], 5001)
    with pytest.raises(ValueError, match="CPU int64"):
        union([torch.tensor([1], dtype=torch.int32)], 10)
    # lists are checked one at a time, dtype then range (cpu_token_union.py:15-20):
    # an out-of-range int64 list ahead of a float list is the range error, and
    # the reverse order is the dtype error
    with pytest.raises(ValueError, match="outside history"):
        union([torch.tensor([12]), torch.tensor([1.0])], 10)
    with pytest.raises(ValueError, match="CPU int64"):
        union([torch.tensor([1.0]), torch.tensor([12])], 10)
    with pytest.raises(ValueError, match="outside history"):
        union([torch.tensor([0])], 0)
