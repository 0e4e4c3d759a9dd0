"""Benchmark of the sparse-decode KV path on one MI355X.

Workload (default): one decode step of a Llama-3-8B-shaped model's
sparse-decode KV path at 32K context with every KV head resident in HBM --
32 layers x (Quest score + top-k + GQA union plan, then the sparse GQA
decode attention over sink ++ union pages ++ recent window ++ decode token,
which also appends the decode token's K/V to the cache).  Per layer:
8 KV heads, 4 query heads per KV head, head_dim 128, fp16, page size 16,
sink 64, recent 256, a Quest budget of 128 pages (2048 tokens) per query
head.  K carries 4 outlier channels (x8) and 16 planted relevant pages per
KV head.  Inputs are synthetic and seeded; each layer has its own K/V,
metadata and queries, so the 32-layer step streams well over the 256 MB
last-level cache.

A "step" is one replay of a HIP graph holding the 32 layers.  ``value`` is
the algorithmic bytes of the step divided by its time (GB/s); ``layer_us`` is
the step time divided by 32.  Per-kernel durations come from graphs holding
only that kernel's 32 launches, timed with events on the launch stream.

The CPU baseline times the oracle's torch-CPU port of the reference's op
sequence for one layer (oracle/cpu_baseline.py) on a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers 32]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "twilight-cpu-gpu-offloading_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "sparse-decode layer µs + achieved GB/s vs roofline; p50 TPOT at 32k ctx"
HBM_PEAK_GBS = 8000.0


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--context", type=int, default=32768)
    ap.add_argument("--budget-pages", type=int, default=128)
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline sample budget (s)")
    ap.add_argument("--calibration-copy", action="store_true",
                    help="also run one 256 MiB device copy (reference kernel for PMC byte counters)")
    return ap.parse_args(argv)


# ---------------------------------------------------------------- inputs
class QuestWorkload:
    """Seeded synthetic inputs of the 32K HBM-resident Quest layer, per layer."""

    G, R, D = 8, 4, 128
    SINK, RECENT, BS = 64, 256, 16
    PLANTED, OUTLIERS = 16, 4

    def __init__(self, dev, layers: int, context: int, budget_pages: int, seed: int = 1):
        import torch

        from headinfer import kernels

        self.dev, self.layers, self.L = dev, layers, context
        G, R, D, L = self.G, self.R, self.D, context
        self.dtype = torch.float16
        self.Lmax = L + 1  # room for the decode token's row
        self.P_meta = (L - self.SINK) // self.BS
        eligible = max(0, max(min(self.SINK, L), L - (self.RECENT - 1)) - min(self.SINK, L))
        self.P = min(eligible // self.BS, self.P_meta)
        self.k = min(budget_pages, self.P)
        self.max_rows = min(self.SINK, L) + min(R * self.k, self.P) * self.BS + (self.RECENT - 1) + 1
        gen = torch.Generator(device=dev).manual_seed(seed)
        f16 = self.dtype
        self.q = torch.randn((layers, G, R, D), generator=gen, device=dev).to(f16)
        self.qf = self.q.float()
        self.kc = torch.empty((layers, G, self.Lmax, D), dtype=f16, device=dev)
        self.vc = torch.empty_like(self.kc)
        self.cur_k = torch.randn((layers, G, D), generator=gen, device=dev).to(f16)
        self.cur_v = torch.randn((layers, G, D), generator=gen, device=dev).to(f16)
        self.pmin = torch.empty((layers, G, self.P_meta, D), dtype=f16, device=dev)
        self.pmax = torch.empty_like(self.pmin)
        for layer in range(layers):
            k = torch.randn((G, self.Lmax, D), generator=gen, device=dev)
            v = torch.randn((G, self.Lmax, D), generator=gen, device=dev)
            # planted pages: keys aligned with the normalised mean query of the group
            u = self.qf[layer].mean(dim=1)
            u = u / u.norm(dim=-1, keepdim=True)
            pages = torch.stack([torch.randperm(self.P, generator=gen, device=dev)[: self.PLANTED] for _ in range(G)])
            rows = (self.SINK + pages.unsqueeze(-1) * self.BS
                    + torch.arange(self.BS, device=dev)).reshape(G, -1)
            noise = torch.randn((G, rows.shape[1], D), generator=gen, device=dev) * 0.1
            k.scatter_(1, rows.unsqueeze(-1).expand(-1, -1, D), 3.0 * u.unsqueeze(1) + noise)
            ch = torch.randperm(D, generator=gen, device=dev)[: self.OUTLIERS]
            k[:, :, ch] *= 8.0
            self.kc[layer].copy_(k.to(f16))
            self.vc[layer].copy_(v.to(f16))
            kernels.build_page_metadata(self.kc[layer, :, :L], sink=self.SINK, block_size=self.BS,
                                        page_min=self.pmin[layer], page_max=self.pmax[layer])
        i32 = torch.int32
        self.max_pages = min(self.P, R * self.k)
        self.plan_pages = torch.zeros((layers, G, self.max_pages), dtype=i32, device=dev)
        self.plan_masks = torch.zeros((layers, G, self.max_pages), dtype=torch.uint8, device=dev)
        self.plan_counts = torch.zeros((layers, G), dtype=i32, device=dev)
        self.sel = torch.zeros((layers, G, R, self.k), dtype=i32, device=dev)
        self.out = torch.empty_like(self.q)
        torch.cuda.synchronize(dev)

    # one layer's kernels -------------------------------------------------
    def select(self, layer: int) -> None:
        from headinfer import kernels

        kernels.quest_select(self.qf[layer], self.pmin[layer, :, : self.P], self.pmax[layer, :, : self.P], self.k,
                             sel_pages=self.sel[layer], plan_pages=self.plan_pages[layer],
                             plan_masks=self.plan_masks[layer], plan_counts=self.plan_counts[layer])

    def append(self, layer: int) -> None:
        from headinfer import kernels

        kernels.append_kv(self.cur_k[layer], self.cur_v[layer], self.kc[layer], self.vc[layer], first_entry=0,
                          position=self.L)

    def attend(self, layer: int) -> None:
        from headinfer import kernels

        kernels.decode_attention_pages(self.q[layer], self.kc[layer], self.vc[layer], self.plan_pages[layer],
                                       self.plan_counts[layer], plan_masks=self.plan_masks[layer],
                                       max_pages=self.max_pages, sink=self.SINK, recent=self.RECENT,
                                       block_size=self.BS, length=self.L, append_position=self.L,
                                       cur_k=self.cur_k[layer], cur_v=self.cur_v[layer], out=self.out[layer])

    def step(self) -> None:
        """One decode step: per layer, Quest selection then attention with the
        decode token's K/V appended to the cache in the same launch."""
        for layer in range(self.layers):
            self.select(layer)
            self.attend(layer)

    # algorithmic bytes ---------------------------------------------------
    def bytes_per_layer(self) -> dict:
        """Algorithmic HBM bytes per layer (mean over layers), by kernel."""
        G, R, D, P, k = self.G, self.R, self.D, self.P, self.k
        e = 2
        fixed = min(self.SINK, self.L) + (self.RECENT - 1) + 1  # sink + recent + the decode token
        rows = (self.plan_counts.double().sum().item() * self.BS + G * fixed) / self.layers
        select = 2 * P * D * e * G + G * R * P * 4 * 2 + G * R * k * 4 + G * R * D * 4
        # K/V rows (the decode token's come from registers), q, out, and the
        # append of the decode token (read + write)
        attention = (rows - G) * 2 * D * e + 2 * G * R * D * e + 4 * G * D * e
        return {"select": select, "attention": attention, "rows_per_group": rows / G}


def graph_of(fn, warm: int = 2):
    import torch

    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_graph(g, reps: int) -> float:
    """Mean seconds per replay, from events on the replay stream."""
    import torch

    s = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    g.replay()
    torch.cuda.synchronize()
    e0.record(s)
    for _ in range(reps):
        g.replay()
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / reps


def check_parity(w: QuestWorkload) -> dict:
    """Size-independent checks on the GPU result of layer 0 (structure of the
    row plan, attention against a float64 recomputation over the same rows)."""
    import numpy as np
    import torch

    G, R, D = w.G, w.R, w.D
    sel = w.sel[0].cpu().numpy()
    ok = bool((np.diff(sel, axis=-1) > 0).all() and sel.min() >= 0 and sel.max() < w.P)
    kc = w.kc[0].float()
    vc = w.vc[0].float()
    err = 0.0
    sink_end = min(w.SINK, w.L)
    recent_start = max(sink_end, w.L - (w.RECENT - 1))
    for g in range(G):
        nu = int(w.plan_counts[0, g])
        pages = w.plan_pages[0, g, :nu].long().cpu()
        pmask = w.plan_masks[0, g, :nu].long().cpu()
        # union plan == union of the per-head selections, masks == heads that chose each page
        ok &= bool(np.array_equal(pages.numpy(), np.unique(sel[g])))
        ok &= all(int(pmask[u]) == sum(1 << r for r in range(R) if int(pages[u]) in sel[g, r]) for u in range(nu))
        bs = w.BS
        rows = torch.cat([torch.arange(sink_end), (w.SINK + pages[:, None] * bs + torch.arange(bs)).reshape(-1),
                          torch.arange(recent_start, w.L), torch.tensor([w.L])]).to(w.q.device)
        all_heads = (1 << R) - 1
        m = torch.cat([torch.full((sink_end,), all_heads), pmask.repeat_interleave(bs),
                       torch.full((w.L - recent_start + 1,), all_heads)]).to(w.q.device)
        s = (kc[g, rows].double() @ w.q[0, g].double().T) / math.sqrt(D)  # [n, R]
        vis = ((m.unsqueeze(1) >> torch.arange(R, device=m.device)) & 1).bool()
        s = s.masked_fill(~vis, float("-inf"))
        p = torch.softmax(s, dim=0)
        ref = p.T @ vc[g, rows].double()
        got = w.out[0, g].double()
        e = (got - ref).abs()
        ok &= bool((e <= 2e-3 + 1e-2 * ref.abs()).all().item())
        err = max(err, float(e.max()))
    return {"ok": ok, "attention_max_abs_err": err}


def cpu_baseline(w: QuestWorkload, seconds: float) -> dict:
    import torch

    from oracle.cpu_baseline import quest_layer_step

    threads = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    L = w.L
    q = w.q[0].cpu()
    kc = w.kc[0, :, :L].cpu()
    vc = w.vc[0, :, :L].cpu()
    pmin = w.pmin[0, :, : w.P].cpu()
    pmax = w.pmax[0, :, : w.P].cpu()
    ck, cv = w.cur_k[0].cpu(), w.cur_v[0].cpu()

    def run():
        return quest_layer_step(q, kc, vc, pmin, pmax, ck, cv, length=L, budget=w.k, sink=w.SINK,
                                recent=w.RECENT, block_size=w.BS)

    run()
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < seconds and len(times) < 200):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(med * 1e6, 1), "unit": "us/layer", "cores": threads, "kind": "port",
            "sample": f"median of {len(times)} single-layer steps (layer 0, all 8 KV heads, torch CPU: "
                      "where/sum score, topk, expand, index_select, SDPA math)"}


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the sparse-decode path of this "
              "build runs on a single MI355X.", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm device", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    from headinfer import _native

    _native.hip()  # fail loudly if the kernel library is missing

    print(f"[bench] building inputs: layers={args.layers} context={args.context}", file=sys.stderr, flush=True)
    w = QuestWorkload(dev, args.layers, args.context, args.budget_pages)

    print("[bench] eager step + parity", file=sys.stderr, flush=True)
    w.step()
    torch.cuda.synchronize()
    parity = check_parity(w)

    if args.calibration_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    print("[bench] capturing graphs", file=sys.stderr, flush=True)
    g_step = graph_of(w.step)
    g_sel = graph_of(lambda: [w.select(i) for i in range(w.layers)])
    g_att = graph_of(lambda: [w.attend(i) for i in range(w.layers)])

    for _ in range(args.warmup):
        g_step.replay()
    torch.cuda.synchronize()
    print(f"[bench] timing {args.steps} steps", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        g_step.replay()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / max(1, args.steps)
    step_event = time_graph(g_step, args.steps)

    reps = max(20, args.steps // 2)
    t_sel = time_graph(g_sel, reps) / w.layers
    t_att = time_graph(g_att, reps) / w.layers
    by = w.bytes_per_layer()
    layer_bytes = by["select"] + by["attention"]
    layer_s = wall / w.layers
    value = layer_bytes / layer_s / 1e9
    kern = {
        "quest_select": {"us": round(t_sel * 1e6, 2), "bytes": int(by["select"]),
                         "GBps": round(by["select"] / t_sel / 1e9, 1)},
        "decode_attention": {"us": round(t_att * 1e6, 2), "bytes": int(by["attention"]),
                             "GBps": round(by["attention"] / t_att / 1e9, 1)},
    }
    dom = "decode_attention" if t_att >= t_sel else "quest_select"
    ach = kern[dom]["GBps"]
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "quest-32k-hbm: Llama-3-8B-shaped sparse-decode KV path, 32 layers x (Quest score + "
                        "top-k + GQA union plan, sparse GQA decode attention with the decode token's K/V "
                        "append), all KV in HBM",
            "layers": w.layers, "context": w.L, "kv_heads": w.G, "q_per_kv": w.R, "head_dim": w.D,
            "page_size": w.BS, "budget_pages": w.k, "scored_pages": w.P, "sink": w.SINK, "recent": w.RECENT,
        },
        "layer_us": round(layer_s * 1e6, 3),
        "layer_us_event": round(step_event / w.layers * 1e6, 3),
        "layer_bytes": int(layer_bytes),
        "step_roofline_frac": round(value / HBM_PEAK_GBS, 4),
        "rows_per_group": round(by["rows_per_group"], 1),
        "union_pages_per_group": round(w.plan_counts.double().mean().item(), 1),
        "kernels": kern,
        "roofline": {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom), "kernel": dom},
        "parity": parity,
    }
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0 if parity["ok"] else 1


# rocprofv3 FETCH_SIZE / WRITE_SIZE of each kernel, calibrated against a copy
# of known size and recorded with the commands that produced them.
TRAFFIC_PROFILE = ROOT / "profiles" / "pmc_traffic_quest32k.md"
TRAFFIC_KERNEL = {"decode_attention": "decode_attn_kernel", "quest_select": "quest_score_kernel"}


def measured_traffic(kernel: str):
    """HBM bytes per launch of the named kernel from the committed PMC
    summary, or None when it is absent."""
    try:
        text = TRAFFIC_PROFILE.read_text()
    except OSError:
        return None
    for line in text.splitlines():
        if line.startswith("traffic_json:"):
            table = json.loads(line.split(":", 1)[1])
            for name, entry in table.items():
                if TRAFFIC_KERNEL.get(kernel, kernel) in name:
                    return int(entry["traffic_bytes"])
    return None


if __name__ == "__main__":
    sys.exit(main())
