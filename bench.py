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
only that kernel's 32 launches (the attention's split-K kernel through the
phase-1 entry point, its merge as the difference to the full call), timed
with events on the launch stream.

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
    ap.add_argument("--workload", choices=("quest32k", "twilight32k", "offload64k", "tpot32k", "multireq"),
                    default="quest32k",
                    help="quest32k (default): 32K layer, KV in HBM; twilight32k: INT4 QK + top-p at 32K; "
                         "offload64k: 64K layer with KV in pinned host memory (zero-copy vs DMA); "
                         "tpot32k: end-to-end p50 TPOT of a Llama-3-8B-shaped model at 32K context; "
                         "multireq: 8 requests of 16K-128K context, Qwen2.5-7B-like GQA, KV heads half in HBM "
                         "and half in host memory, 256 decode steps with append and metadata update")
    ap.add_argument("--decode-tokens", type=int, default=32, help="decode tokens per TPOT run (D1..Dn)")
    ap.add_argument("--tpot-only", default=None,
                    help="tpot32k: run this variant only (e.g. sparse_graph, for a profile of its kernels)")
    ap.add_argument("--kv-residency", choices=("hbm", "host"), default="hbm",
                    help="tpot32k: KV slab in HBM or in pinned host memory (read zero-copy)")
    ap.add_argument("--context", type=int, default=None, help="context length (workload default if omitted)")
    ap.add_argument("--budget-mode", choices=("dynamic", "matched"), default="dynamic",
                    help="Twilight budgets (twilight32k)")
    ap.add_argument("--budget-pages", type=int, default=128)
    ap.add_argument("--twilight-path", choices=("fused", "pages", "rows"), default="fused",
                    help="Twilight selection + union form: fused (score + one per-head launch, union record), "
                         "pages (B0 plan, INT4 QK, top-p into B0 union page row masks) or rows (union row list)")
    ap.add_argument("--union", choices=("bits", "plan"), default="bits",
                    help="quest32k: the GQA union as per-head selection bitmaps ranked by the attention (bits) "
                         "or as a union plan built after the top-k (plan)")
    ap.add_argument("--requests", type=int, default=1,
                    help="quest32k: decode this many requests of the same context per launch (8 KV groups each)")
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-host-tpot", action="store_true",
                    help="default workload: leave out the 64K pinned-host TPOT leg")
    ap.add_argument("--quest-only", action="store_true",
                    help="default workload: only the Quest 32K leg (no Twilight / host-offload / TPOT summaries)")
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

    def __init__(self, dev, layers: int, context: int, budget_pages: int, seed: int = 1, requests: int = 1,
                 union: str = "bits", planted: int | None = None, outliers: int | None = None):
        import torch

        from headinfer import kernels

        self.dev, self.layers, self.L = dev, layers, context
        # the 32K layer's structure by default; the 4K layer has 4 planted
        # pages and no outlier channels
        self.PLANTED = type(self).PLANTED if planted is None else planted
        self.OUTLIERS = type(self).OUTLIERS if outliers is None else outliers
        # "bits": per-head selection bitmaps ranked by the attention; "plan":
        # the union plan built by the top-k's last block of each group
        self.union = union
        # a batch of requests at one context length: every request's KV groups
        # side by side in the same launches
        self.requests = requests
        self.G = type(self).G * requests
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
        self.bits = torch.zeros((layers, G, R, kernels.sel_bits_words(self.P)), dtype=i32, device=dev)
        if self.union == "bits" and self.P > 8192:
            self.union = "plan"  # longer rows select through the segment pass and a plan
        self.out = torch.empty_like(self.q)
        torch.cuda.synchronize(dev)

    # one layer's kernels -------------------------------------------------
    def select(self, layer: int) -> None:
        from headinfer import kernels

        if self.union == "bits":
            kernels.quest_select_bits(self.qf[layer], self.pmin[layer, :, : self.P], self.pmax[layer, :, : self.P],
                                      self.k, self.bits[layer])
            return
        kernels.quest_select(self.qf[layer], self.pmin[layer, :, : self.P], self.pmax[layer, :, : self.P], self.k,
                             sel_pages=self.sel[layer], plan_pages=self.plan_pages[layer],
                             plan_masks=self.plan_masks[layer], plan_counts=self.plan_counts[layer])

    def union_of(self, layer: int, g: int):
        """(ascending union pages, head masks) of group g at `layer` from the
        selection the step produced."""
        import numpy as np

        if self.union == "bits":
            w = self.bits[layer, g].cpu().numpy().view(np.uint32)
            p = np.arange(self.P)
            hb = ((w[:, p >> 5] >> (p & 31).astype(np.uint32)) & 1).astype(np.int64)  # [R, P]
            pages = np.flatnonzero(hb.any(axis=0))
            masks = (hb[:, pages] << np.arange(self.R)[:, None]).sum(axis=0)
            return pages, masks
        nu = int(self.plan_counts[layer, g])
        return (self.plan_pages[layer, g, :nu].long().cpu().numpy(),
                self.plan_masks[layer, g, :nu].long().cpu().numpy())

    def union_counts(self):
        """Union pages per (layer, group)."""
        import torch

        if self.union == "bits":
            b = self.bits.view(torch.int32).cpu()
            words = b[..., 0::2].long() & 0xffffffff | (b[..., 1::2].long() << 32)
            u = words[:, :, 0]
            for r in range(1, self.R):
                u = u | words[:, :, r]
            return torch.tensor([[sum(bin(int(x) & 0xffffffffffffffff).count("1") for x in u[l, g])
                                  for g in range(self.G)] for l in range(self.layers)], dtype=torch.float64)
        return self.plan_counts.double().cpu()

    def selection_of(self, layer: int):
        """Every head's selected pages at `layer` (ascending arrays, [G][R]),
        read from what the timed step wrote: the selection bitmaps, or the
        per-head page lists of the plan form."""
        import numpy as np

        if self.union == "bits":
            w = self.bits[layer].cpu().numpy().view(np.uint32)
            p = np.arange(self.P)
            hb = ((w[:, :, p >> 5] >> (p & 31).astype(np.uint32)) & 1).astype(bool)   # [G, R, P]
            return [[np.flatnonzero(hb[g, r]) for r in range(self.R)] for g in range(self.G)]
        sel = self.sel[layer].long().cpu().numpy()
        return [[sel[g, r] for r in range(self.R)] for g in range(self.G)]

    def append(self, layer: int) -> None:
        from headinfer import kernels

        kernels.append_kv(self.cur_k[layer], self.cur_v[layer], self.kc[layer], self.vc[layer], first_entry=0,
                          position=self.L)

    def attend(self, layer: int, phase: int = 3) -> None:
        from headinfer import kernels

        if self.union == "bits":
            kernels.decode_attention_pages_bits(self.q[layer], self.kc[layer], self.vc[layer], self.bits[layer], self.P,
                                                max_pages=self.max_pages, sink=self.SINK, recent=self.RECENT,
                                                block_size=self.BS, length=self.L, append=True,
                                                cur_k=self.cur_k[layer], cur_v=self.cur_v[layer],
                                                out=self.out[layer], phase=phase)
            return
        kernels.decode_attention_pages(self.q[layer], self.kc[layer], self.vc[layer], self.plan_pages[layer],
                                       self.plan_counts[layer], plan_masks=self.plan_masks[layer],
                                       max_pages=self.max_pages, sink=self.SINK, recent=self.RECENT,
                                       block_size=self.BS, length=self.L, append_position=self.L,
                                       cur_k=self.cur_k[layer], cur_v=self.cur_v[layer], out=self.out[layer],
                                       phase=phase)

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
        rows = (self.union_counts().sum().item() * self.BS + G * fixed) / self.layers
        select = 2 * P * D * e * G + G * R * P * 4 * 2 + G * R * k * 4 + G * R * D * 4
        # K/V rows (the decode token's come from registers), q, out, and the
        # append of the decode token (read + write)
        attention = (rows - G) * 2 * D * e + 2 * G * R * D * e + 4 * G * D * e
        return {"select": select, "attention": attention, "rows_per_group": rows / G}


class TwilightWorkload:
    """Seeded synthetic inputs of the 32K Twilight layer: bf16 K/V in HBM,
    per-token INT4 keys, Quest B0 = 4096 tokens (256 pages), top-p 0.95 with
    dynamic budgets, page relevance Zipf(1.1) over permuted ranks added as
    4 * w_p * u_g to the page's keys (u_g the normalised mean query)."""

    G, R, D = 8, 4, 128
    SINK, RECENT, BS = 64, 256, 16
    B0_TOKENS, TOP_P, ALPHA, ZIPF = 4096, 0.95, 4.0, 1.1

    def __init__(self, dev, layers: int, context: int, budget_mode: str = "dynamic", seed: int = 2,
                 path: str = "fused"):
        import torch

        from headinfer import kernels

        self.dev, self.layers, self.L, self.mode = dev, layers, context, budget_mode
        G, R, D, L = self.G, self.R, self.D, context
        bf = torch.bfloat16
        self.Lmax = L + 1
        self.P_meta = (L - self.SINK) // self.BS
        sink_end = min(self.SINK, L)
        recent_start = max(sink_end, L - (self.RECENT - 1))
        self.P = min((recent_start - sink_end) // self.BS, self.P_meta)
        self.b0 = min(self.P, self.B0_TOKENS // self.BS)
        self.N = self.b0 * self.BS
        self.fixed = min(self.P, max(1, math.ceil(0.05 * (recent_start - sink_end) / self.BS)))
        gen = torch.Generator(device=dev).manual_seed(seed)
        self.q = torch.randn((layers, G, R, D), generator=gen, device=dev).to(bf)
        self.qf = self.q.float()
        self.kc = torch.empty((layers, G, self.Lmax, D), dtype=bf, device=dev)
        self.vc = torch.empty_like(self.kc)
        self.cur_k = torch.randn((layers, G, D), generator=gen, device=dev).to(bf)
        self.cur_v = torch.randn((layers, G, D), generator=gen, device=dev).to(bf)
        self.pmin = torch.empty((layers, G, self.P_meta, D), dtype=bf, device=dev)
        self.pmax = torch.empty_like(self.pmin)
        self.packed = torch.empty((layers, G, self.Lmax, D // 2), dtype=torch.uint8, device=dev)
        self.scale = torch.empty((layers, G, self.Lmax), dtype=bf, device=dev)
        self.minimum = torch.empty_like(self.scale)
        ranks = torch.arange(1, self.P + 1, device=dev, dtype=torch.float32)
        for layer in range(layers):
            k = torch.randn((G, self.Lmax, D), generator=gen, device=dev)
            u = self.qf[layer].mean(dim=1)
            u = u / u.norm(dim=-1, keepdim=True)
            for g in range(G):
                w = ranks[torch.randperm(self.P, generator=gen, device=dev)] ** (-self.ZIPF)
                rows = self.SINK + torch.arange(self.P * self.BS, device=dev)
                k[g, rows] += self.ALPHA * w.repeat_interleave(self.BS).unsqueeze(1) * u[g]
            self.kc[layer].copy_(k.to(bf))
            self.vc[layer].copy_(torch.randn((G, self.Lmax, D), generator=gen, device=dev).to(bf))
            kernels.build_page_metadata(self.kc[layer, :, :L], sink=self.SINK, block_size=self.BS,
                                        page_min=self.pmin[layer], page_max=self.pmax[layer],
                                        packed=self.packed[layer], scale=self.scale[layer],
                                        minimum=self.minimum[layer])
        i32 = torch.int32
        self.width = min(self.P, R * self.b0)
        self.sel = torch.zeros((layers, G, R, self.b0), dtype=i32, device=dev)
        self.plan_pages = torch.zeros((layers, G, self.width), dtype=i32, device=dev)
        self.plan_masks = torch.zeros((layers, G, self.width), dtype=torch.uint8, device=dev)
        self.plan_counts = torch.zeros((layers, G), dtype=i32, device=dev)
        self.logits = torch.empty((layers, G, R, self.N), dtype=torch.float32, device=dev)
        self.rows = torch.zeros((layers, G, self.Lmax), dtype=i32, device=dev)
        self.row_counts = torch.zeros((layers, G), dtype=i32, device=dev)
        self.desired = torch.zeros((layers, G, R), dtype=i32, device=dev)
        self.max_rows = min(L, sink_end + R * self.N + (L - recent_start))
        self.out = torch.empty_like(self.q)
        # dynamic budgets: the kept rows as row masks of the B0 union pages,
        # attended page by page (the same rows as the union row list)
        self.page_rows = budget_mode == "dynamic" and path == "pages"
        self.slot_u = torch.zeros((layers, G, R, self.b0), dtype=i32, device=dev)
        self.prows = torch.zeros((layers, G, self.width), dtype=i32, device=dev)
        # fused: two selection launches (score; per-head B0 + INT4 QK + top-p)
        # writing each group's union record, and with matched budgets a third
        # (allocation and each head's top-allocated rows)
        self.fused = path == "fused"
        self.path = path if budget_mode == "dynamic" or path == "fused" else "rows"
        words = (kernels.union_record_words(self.P) + 3) & ~3
        self.rec = torch.zeros((layers, G, words), dtype=i32, device=dev)
        torch.cuda.synchronize(dev)

    def select(self, layer: int, phase: int = 3) -> None:
        from headinfer import kernels

        if self.fused:
            kernels.twilight_select_fused(self.qf[layer], self.pmin[layer, :, : self.P], self.pmax[layer, :, : self.P],
                                          self.packed[layer], self.scale[layer], self.minimum[layer], self.b0,
                                          self.rec[layer], top_p=self.TOP_P, sink=self.SINK, recent=self.RECENT,
                                          block_size=self.BS, length=self.L, desired=self.desired[layer],
                                          budget_mode=self.mode,
                                          target_total=self.fixed * self.BS * self.R if self.mode == "matched" else 0,
                                          phase=phase)
            return
        kernels.quest_select(self.qf[layer], self.pmin[layer, :, : self.P], self.pmax[layer, :, : self.P], self.b0,
                             sel_pages=self.sel[layer], plan_pages=self.plan_pages[layer],
                             plan_masks=self.plan_masks[layer], plan_counts=self.plan_counts[layer])
        pr = dict(slot_u=self.slot_u[layer], page_rows=self.prows[layer]) if self.page_rows else {}
        kernels.twilight_qk(self.qf[layer], self.packed[layer], self.scale[layer], self.minimum[layer],
                            self.plan_pages[layer], self.plan_masks[layer], self.plan_counts[layer], self.b0,
                            sink=self.SINK, block_size=self.BS, out=self.logits[layer], **pr)
        if self.page_rows:
            kernels.twilight_select_pages(self.logits[layer], self.sel[layer], self.slot_u[layer], self.prows[layer],
                                          top_p=self.TOP_P, sink=self.SINK, recent=self.RECENT, block_size=self.BS,
                                          length=self.L, desired=self.desired[layer])
            return
        kernels.twilight_select(self.logits[layer], self.sel[layer], top_p=self.TOP_P, budget_mode=self.mode,
                                target_total=self.fixed * self.BS * self.R, rows=self.rows[layer],
                                row_counts=self.row_counts[layer], desired=self.desired[layer], sink=self.SINK,
                                recent=self.RECENT, block_size=self.BS, length=self.L)

    def attend(self, layer: int, phase: int = 3) -> None:
        from headinfer import kernels

        if self.fused:
            kernels.decode_attention_union(self.q[layer], self.kc[layer], self.vc[layer], self.rec[layer], self.P,
                                           max_pages=self.width, sink=self.SINK, recent=self.RECENT,
                                           block_size=self.BS, length=self.L, append=True, cur_k=self.cur_k[layer],
                                           cur_v=self.cur_v[layer], out=self.out[layer], phase=phase)
            return
        if self.page_rows:
            kernels.decode_attention_page_rows(self.q[layer], self.kc[layer], self.vc[layer], self.plan_pages[layer],
                                               self.plan_counts[layer], self.prows[layer], max_pages=self.width,
                                               sink=self.SINK, recent=self.RECENT, block_size=self.BS, length=self.L,
                                               append=True, cur_k=self.cur_k[layer], cur_v=self.cur_v[layer],
                                               out=self.out[layer])
            return
        kernels.decode_attention_rows(self.q[layer], self.kc[layer], self.vc[layer], self.rows[layer],
                                      self.row_counts[layer], self.max_rows, cur_k=self.cur_k[layer],
                                      cur_v=self.cur_v[layer], out=self.out[layer], append_position=self.L)

    def kept_rows(self, layer: int, g: int):
        """Token positions group g attends at `layer` (without the decode
        token), ascending."""
        import torch

        sink_end = min(self.SINK, self.L)
        recent_start = max(sink_end, self.L - (self.RECENT - 1))
        if self.fused:
            rec = self.rec[layer, g].long() & 0xFFFFFFFF
            off = ((2 * ((self.P + 63) // 64)) + 3) & ~3
            dev = rec.device
            pages = torch.arange(self.P, device=dev)
            masks = (rec[off + (pages >> 1)] >> (16 * (pages & 1))) & 0xFFFF
            bits = (masks[:, None] >> torch.arange(self.BS, device=dev)) & 1
            pos = self.SINK + pages[:, None] * self.BS + torch.arange(self.BS, device=dev)
            return torch.cat([torch.arange(sink_end, device=dev), pos[bits.bool()],
                              torch.arange(recent_start, self.L, device=dev)])
        if not self.page_rows:
            n = int(self.row_counts[layer, g])
            return self.rows[layer, g, :n].long()
        nu = int(self.plan_counts[layer, g])
        pages = self.plan_pages[layer, g, :nu].long()
        masks = self.prows[layer, g, :nu].long() & 0xFFFFFFFF
        bits = (masks[:, None] >> torch.arange(self.BS, device=masks.device)) & 1
        pos = self.SINK + pages[:, None] * self.BS + torch.arange(self.BS, device=masks.device)
        dev = masks.device
        return torch.cat([torch.arange(sink_end, device=dev), pos[bits.bool()],
                          torch.arange(recent_start, self.L, device=dev)])

    def step(self) -> None:
        for layer in range(self.layers):
            self.select(layer)
            self.attend(layer)

    def candidate_union_rows(self) -> float:
        """Sum over groups of |C_g|, the union of the group's per-head B0
        candidate rows (mean over layers), measured: the B0 pages are the
        Quest top-b0 of each head, the same pages the selection launches
        take, listed here by a separate top-k outside any timed region."""
        import numpy as np

        from headinfer import kernels

        total = 0
        for layer in range(self.layers):
            kernels.quest_select(self.qf[layer], self.pmin[layer, :, : self.P], self.pmax[layer, :, : self.P],
                                 self.b0, sel_pages=self.sel[layer])
            sel = self.sel[layer].cpu().numpy()
            total += sum(np.unique(sel[g]).size for g in range(self.G)) * self.BS
        return total / self.layers

    def bytes_per_layer(self) -> dict:
        """Algorithmic HBM bytes per layer (mean over layers) by stage, as the
        scope's measurement defines them: page min/max once per group, the
        scores and the candidates' logits written and read back, the INT4
        rows (codes, scale, minimum) of Sum_g |C_g| candidates (the union of
        the heads' candidate sets), the attended K/V rows, q and the output.
        The fused selection reads the INT4 rows of every scored page (more
        than Sum_g |C_g|); that excess is traffic, not algorithmic bytes."""
        G, R, D, P, N = self.G, self.R, self.D, self.P, self.N
        e = 2
        if self.page_rows or self.fused:                                            # attended union rows
            rows = sum(self.kept_rows(layer, g).numel() for layer in range(self.layers) for g in range(G)) / self.layers
        else:
            rows = self.row_counts.double().sum().item() / self.layers
        if self.fused:
            cand_rows = self.candidate_union_rows()
        else:
            cand_rows = self.plan_counts.double().sum().item() * self.BS / self.layers   # union of the B0 candidates
        int4 = cand_rows * (D // 2 + 2 * e)
        score = 2 * P * D * e * G + G * R * P * 4 + G * R * D * 4      # metadata + q in, scores out
        if self.fused:
            # the score + QK launch also reads the candidates' INT4 rows and
            # writes their logits; the head launch reads the scores and those
            # logits back and ORs the union records
            score += int4 + G * R * N * 4
            head = G * R * P * 4 + G * R * N * 4 + G * self.rec.shape[2] * 4
            if self.mode == "matched":  # the allocation launch reads the logits back
                head += G * R * N * 4 * 2
        else:
            head = G * R * P * 4 + G * R * self.b0 * 4 + int4 + G * R * N * 4 * 2
        attention = rows * 2 * D * e + 2 * G * R * D * e + 4 * G * D * e
        return {"select": score + head, "score": score, "head": head, "attention": attention,
                "rows_per_group": rows / G, "candidate_rows_per_group": cand_rows / G,
                "per_head_candidate_rows_per_group": R * N}


class OffloadWorkload(QuestWorkload):
    """The 64K layer with every KV head in pinned host memory (page metadata
    in HBM): Quest selection on the GPU, then the sparse attention reading the
    selected pages either zero-copy over the host link (mapped pinned memory)
    or after a host gather into pinned staging and one DMA copy."""

    def __init__(self, dev, layers: int, context: int, budget_pages: int, seed: int = 3):
        import torch

        super().__init__(dev, layers, context, budget_pages, seed=seed, union="plan")  # the DMA leg reads the plan
        hk = torch.empty(self.kc.shape, dtype=self.kc.dtype, pin_memory=True)
        hv = torch.empty(self.vc.shape, dtype=self.vc.dtype, pin_memory=True)
        hk.copy_(self.kc)
        hv.copy_(self.vc)
        self.hk, self.hv = hk, hv
        del self.kc, self.vc
        torch.cuda.empty_cache()
        G, D = self.G, self.D
        self.dev_k = torch.empty((G, self.max_rows, D), dtype=hk.dtype, device=dev)
        self.dev_v = torch.empty_like(self.dev_k)
        self.rmask_h = torch.zeros((G, self.max_rows), dtype=torch.uint8, pin_memory=True)
        self.counts_h = torch.zeros((G,), dtype=torch.int32, pin_memory=True)
        self.rows_d = torch.zeros((G, self.max_rows), dtype=torch.int32, device=dev)
        self.rmask_d = torch.zeros((G, self.max_rows), dtype=torch.uint8, device=dev)
        self.counts_d = torch.zeros((G,), dtype=torch.int32, device=dev)

    def attend(self, layer: int) -> None:
        from headinfer import kernels

        kernels.decode_attention_pages(self.q[layer], self.hk[layer], self.hv[layer], self.plan_pages[layer],
                                       self.plan_counts[layer], plan_masks=self.plan_masks[layer],
                                       max_pages=self.max_pages, sink=self.SINK, recent=self.RECENT,
                                       block_size=self.BS, length=self.L, append_position=self.L,
                                       cur_k=self.cur_k[layer], cur_v=self.cur_v[layer], out=self.out[layer])

    def attend_dma(self, layer: int, groups_per_chunk: int = 2) -> int:
        """The DMA alternative to zero-copy (the reference's post-selection
        pipeline, twilight_offload_cache.py:2053-2455): the layer's union
        plans come to the host in one copy, then chunk by chunk the CPU
        gathers the union rows from the pinned slab into pinned staging and a
        side stream copies them to HBM, while the next chunk is gathered; each
        chunk's attention over its staged rows starts behind its copy.
        Returns the rows moved."""
        import numpy as np
        import torch

        from headinfer import kernels
        from headinfer.dma_pipeline import HostGatherPipeline

        plan = torch.cat([self.plan_counts[layer].view(-1, 1), self.plan_pages[layer],
                          self.plan_masks[layer].to(torch.int32)], dim=1).cpu().numpy()
        G, R, BS, L, D = self.G, self.R, self.BS, self.L, self.D
        W = self.plan_pages.shape[2]
        sink_end = min(self.SINK, L)
        recent_start = max(sink_end, L - (self.RECENT - 1))
        n_fixed = sink_end + (L - recent_start)
        if getattr(self, "dma", None) is None:
            self.dma = HostGatherPipeline(self.dev, D, self.hk.dtype, groups_per_chunk * self.max_rows)
            self.rows_d.copy_(torch.arange(self.max_rows, dtype=torch.int32).expand(G, -1))
            head = np.full(sink_end, (1 << R) - 1, np.uint8)
            tail = np.full(L - recent_start, (1 << R) - 1, np.uint8)
            self._dma_fixed = (np.arange(sink_end, dtype=np.int64), np.arange(recent_start, L, dtype=np.int64),
                               head, tail)
        sink_pos, recent_pos, head, tail = self._dma_fixed
        counts = plan[:, 0]
        n = counts * BS + n_fixed
        offs = np.arange(BS, dtype=np.int64)
        rmask = np.zeros((G, self.max_rows), np.uint8)
        dst_k = self.dev_k.view(-1, D)
        dst_v = self.dev_v.view(-1, D)
        chunks = []
        for c0 in range(0, G, groups_per_chunk):
            ids = []
            for g in range(c0, min(G, c0 + groups_per_chunk)):
                nu = int(counts[g])
                body = (self.SINK + plan[g, 1:1 + nu].astype(np.int64)[:, None] * BS + offs).reshape(-1)
                base = g * self.Lmax
                ids.append(np.concatenate([sink_pos, body, recent_pos]) + base)
                pad = self.max_rows - int(n[g])  # staged groups sit max_rows apart
                if pad:
                    ids.append(np.full(pad, base, np.int64))
                rmask[g, :n[g]] = np.concatenate([head, np.repeat(plan[g, 1 + W:1 + W + nu].astype(np.uint8), BS),
                                                  tail])
            ids = np.concatenate(ids)
            a = c0 * self.max_rows
            chunks.append((ids, dst_k[a:a + ids.shape[0]], dst_v[a:a + ids.shape[0]]))
        self.counts_d.copy_(torch.from_numpy(n.astype(np.int32)), non_blocking=False)
        self.rmask_d.copy_(torch.from_numpy(rmask), non_blocking=False)

        def attend(c: int) -> None:
            g0, g1 = c * groups_per_chunk, min(G, (c + 1) * groups_per_chunk)
            kernels.decode_attention_rows(self.q[layer, g0:g1], self.dev_k[g0:g1], self.dev_v[g0:g1],
                                          self.rows_d[g0:g1], self.counts_d[g0:g1], self.max_rows,
                                          row_masks=self.rmask_d[g0:g1], cur_k=self.cur_k[layer, g0:g1],
                                          cur_v=self.cur_v[layer, g0:g1], out=self.out[layer, g0:g1])

        self.dma.run(self.hk[layer].view(-1, D), self.hv[layer].view(-1, D), chunks, on_chunk=attend)
        kernels.append_kv(self.cur_k[layer], self.cur_v[layer], self.hk[layer], self.hv[layer], first_entry=0,
                          position=self.L)
        return int(n.sum())

    def host_bytes_per_layer(self) -> float:
        fixed = min(self.SINK, self.L) + (self.RECENT - 1)
        rows = self.plan_counts.double().sum().item() * self.BS / self.layers + self.G * fixed
        return rows * 2 * self.D * 2 + self.G * 2 * self.D * 2  # selected K/V rows read + decode token written


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

    from headinfer import kernels

    G, R, D = w.G, w.R, w.D
    if w.union == "bits":
        # the per-head page lists of the same selection, for the set checks
        kernels.quest_select(w.qf[0], w.pmin[0, :, : w.P], w.pmax[0, :, : w.P], w.k, sel_pages=w.sel[0])
        torch.cuda.synchronize()
    sel = w.sel[0].cpu().numpy()
    ok = bool((np.diff(sel, axis=-1) > 0).all() and sel.min() >= 0 and sel.max() < w.P)
    kc = w.kc[0].float()
    vc = w.vc[0].float()
    err = 0.0
    sink_end = min(w.SINK, w.L)
    recent_start = max(sink_end, w.L - (w.RECENT - 1))
    for g in range(G):
        pages_np, masks_np = w.union_of(0, g)
        nu = pages_np.shape[0]
        pages = torch.from_numpy(pages_np).long()
        pmask = torch.from_numpy(masks_np).long()
        # union == union of the per-head selections, masks == heads that chose each page
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


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _bits(t):
    """A 16-bit float tensor's storage as uint16 (the oracle's input form)."""
    import numpy as np
    import torch

    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _sampled(run, budget_s: float, cap: int) -> tuple[float, int]:
    """Median seconds of run() over a bounded sample (at least 3 calls, then
    until budget_s or cap calls), after one untimed call."""
    run()
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < cap):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def quest_oracle_check(w: QuestWorkload, layer: int = 0) -> dict:
    """Verification of the CPU-baseline leg: every head's pages the timed step
    selected at `layer` against oracle.topk_sorted(oracle.quest_score(...))
    (bit for bit, quest_offload_cache.py:362-374), and each head's attention
    output within 2e-3 abs + 1e-2 rel of float64 over sink ++ the oracle's
    pages ++ recent ++ the decode token."""
    import numpy as np
    import torch

    import oracle

    G, R, D, P, L = w.G, w.R, w.D, w.P, w.L
    q = w.qf[layer].cpu().numpy()
    sc = oracle.quest_score(q, _bits(w.pmin[layer, :, :P]), _bits(w.pmax[layer, :, :P]), "f16")
    want = oracle.topk_sorted(sc.reshape(G * R, P), w.k).reshape(G, R, w.k)
    got = w.selection_of(layer)
    match = all(np.array_equal(got[g][r], want[g, r]) for g in range(G) for r in range(R))
    sink_end, recent_start, _ = oracle.selection_window(L, w.SINK, w.RECENT)
    kc, vc = w.kc[layer].cpu().float(), w.vc[layer].cpu().float()
    out = w.out[layer].float().cpu().numpy()
    err, att_ok = 0.0, True
    for g in range(G):
        for r in range(R):
            pages = torch.from_numpy(want[g, r]).long()
            rows = torch.cat([torch.arange(sink_end), (w.SINK + pages[:, None] * w.BS + torch.arange(w.BS)).reshape(-1),
                              torch.arange(recent_start, L)])
            keys = torch.cat([kc[g, rows], w.cur_k[layer, g:g + 1].cpu().float()]).numpy()
            vals = torch.cat([vc[g, rows], w.cur_v[layer, g:g + 1].cpu().float()]).numpy()
            ref = oracle.decode_attention(q[g, r:r + 1], keys, vals, 1.0 / math.sqrt(D))[0]
            e = np.abs(out[g, r].astype(np.float64) - ref)
            att_ok &= bool(np.all(e <= 2e-3 + 1e-2 * np.abs(ref)))
            err = max(err, float(e.max()))
    return {"ok": bool(match and att_ok), "selection_match": bool(match), "heads": G * R, "layer": layer,
            "attention_max_abs_err": err,
            "verified_against": "oracle.quest_score + oracle.topk_sorted (pages, bit for bit); float64 attention over "
                       "the oracle's rows"}


def cpu_baseline(w: QuestWorkload, seconds: float) -> dict:
    """The torch-CPU port of the reference's Quest layer step, on this box's
    host cores: with every core of the process's affinity (the headline) and
    with 6 threads (the reference's formal runs), median over a bounded sample,
    with the time split into score + top-k, row gather and attention.  The
    leg also checks layer 0 of the timed step against the oracle."""
    import torch

    from oracle.cpu_baseline import quest_layer_step

    L = w.L
    q = w.q[0].cpu()
    kc = w.kc[0, :, :L].cpu()
    vc = w.vc[0, :, :L].cpu()
    pmin = w.pmin[0, :, : w.P].cpu()
    pmax = w.pmax[0, :, : w.P].cpu()
    ck, cv = w.cur_k[0].cpu(), w.cur_v[0].cpu()
    threads0 = torch.get_num_threads()

    def sample(threads: int, budget_s: float) -> dict:
        torch.set_num_threads(threads)
        phases: dict = {}
        calls = [0]

        def run():
            calls[0] += 1
            return quest_layer_step(q, kc, vc, pmin, pmax, ck, cv, length=L, budget=w.k, sink=w.SINK,
                                    recent=w.RECENT, block_size=w.BS, phases=phases)

        med, n = _sampled(run, budget_s, 200)
        return {"us_per_layer": round(med * 1e6, 1), "steps": n,
                "phases_us": {k: round(v / calls[0] * 1e6, 1) for k, v in phases.items()}}

    n_aff = len(os.sched_getaffinity(0))
    full = sample(n_aff, seconds)
    six = sample(6, seconds / 2)
    torch.set_num_threads(threads0)
    return {"value": full["us_per_layer"], "unit": "us/layer", "cores": n_aff, "kind": "port",
            "sample": f"median of {full['steps']} single-layer steps (layer 0, all {w.G} KV heads, {L // 1024}K "
                      f"context, k = {w.k} pages, torch CPU: where/sum score, topk, expand, index_select, SDPA math)",
            "cpu_model": _cpu_model(), "phases_us": full["phases_us"],
            "threads_6": {"value": six["us_per_layer"], "phases_us": six["phases_us"], "steps": six["steps"]},
            "oracle_check": quest_oracle_check(w, 0)}


def twilight_oracle_check(w: "TwilightWorkload", layer: int = 0) -> dict:
    """Verification of the Twilight CPU-baseline leg: for every group of
    `layer`, the rows the timed step kept (its union record) == the union of
    oracle.twilight_layer, the top-p counts equal, and the union attention
    within 2e-3 abs + 1e-2 rel of float64 over the oracle's rows plus the
    decode token (twilight_offload_cache.py:1144-1354)."""
    import numpy as np
    import torch

    import oracle

    G, D, P, L = w.G, w.D, w.P, w.L
    union_ok = counts_ok = att_ok = True
    err = 0.0
    out = w.out[layer].float().cpu().numpy()
    des = w.desired[layer].cpu().numpy()
    kc, vc = w.kc[layer].cpu().float(), w.vc[layer].cpu().float()
    for g in range(G):
        ref = oracle.twilight_layer(w.qf[layer, g].cpu().numpy(), _bits(w.pmin[layer, g, :P]),
                                    _bits(w.pmax[layer, g, :P]), w.packed[layer, g].cpu().numpy(),
                                    _bits(w.scale[layer, g]), _bits(w.minimum[layer, g]), "bf16", length=L,
                                    sink=w.SINK, recent=w.RECENT, block_size=w.BS, b0_pages=w.b0, top_p=w.TOP_P,
                                    budget_mode=w.mode, fixed_pages=w.fixed)
        counts_ok &= bool(np.array_equal(des[g], ref["desired"]))
        union_ok &= bool(np.array_equal(w.kept_rows(layer, g).cpu().numpy(), ref["union"]))
        rows = torch.from_numpy(ref["union"].astype(np.int64))
        keys = torch.cat([kc[g, rows], w.cur_k[layer, g:g + 1].cpu().float()]).numpy()
        vals = torch.cat([vc[g, rows], w.cur_v[layer, g:g + 1].cpu().float()]).numpy()
        ref_o = oracle.decode_attention(w.qf[layer, g].cpu().numpy(), keys, vals, 1.0 / math.sqrt(D))
        e = np.abs(out[g].astype(np.float64) - ref_o)
        att_ok &= bool(np.all(e <= 2e-3 + 1e-2 * np.abs(ref_o)))
        err = max(err, float(e.max()))
    return {"ok": bool(union_ok and counts_ok and att_ok), "union_match": union_ok, "top_p_counts_match": counts_ok,
            "groups": G, "layer": layer, "attention_max_abs_err": err,
            "verified_against": "oracle.twilight_layer (B0 pages, INT4 QK, exact top-p, allocation, union); float64 "
                       "attention over the oracle's rows"}


def twilight_cpu_baseline(w: "TwilightWorkload", seconds: float) -> dict:
    """The torch-CPU port of the reference's Twilight layer step
    (oracle/cpu_baseline.py twilight_layer_step, dynamic or matched budgets
    as the workload) on layer 0's inputs, with every core of the process's
    affinity and with 6 threads, median over a bounded sample, with the time
    split into phases; plus the oracle check of the timed step's layer 0."""
    import torch

    from oracle.cpu_baseline import twilight_layer_step

    L = w.L
    cpu = [t.cpu() for t in (w.q[0], w.kc[0, :, :L], w.vc[0, :, :L], w.pmin[0, :, : w.P], w.pmax[0, :, : w.P],
                             w.packed[0], w.scale[0], w.minimum[0], w.cur_k[0], w.cur_v[0])]
    threads0 = torch.get_num_threads()

    def sample(threads: int, budget_s: float) -> dict:
        torch.set_num_threads(threads)
        phases: dict = {}
        calls = [0]

        def run():
            calls[0] += 1
            twilight_layer_step(*cpu, length=L, b0_pages=w.b0, top_p=w.TOP_P, sink=w.SINK, recent=w.RECENT,
                                block_size=w.BS, budget_mode=w.mode, fixed_pages=w.fixed, phases=phases)

        med, n = _sampled(run, budget_s, 100)
        return {"us_per_layer": round(med * 1e6, 1), "steps": n,
                "phases_us": {k: round(v / calls[0] * 1e6, 1) for k, v in phases.items()}}

    n_aff = len(os.sched_getaffinity(0))
    full = sample(n_aff, seconds)
    six = sample(6, seconds / 2)
    torch.set_num_threads(threads0)
    return {"value": full["us_per_layer"], "unit": "us/layer", "cores": n_aff, "kind": "port",
            "sample": f"median of {full['steps']} single-layer steps (layer 0, {w.G} KV heads, {L // 1024}K "
                      f"context, B0 {w.N} tokens, top-p {w.TOP_P}, {w.mode} budgets; torch CPU: score, topk, "
                      "INT4 dequant + matmul, argsort/softmax/cumsum top-p, union, index_select, SDPA)",
            "cpu_model": _cpu_model(), "phases_us": full["phases_us"],
            "threads_6": {"value": six["us_per_layer"], "phases_us": six["phases_us"], "steps": six["steps"]},
            "oracle_check": twilight_oracle_check(w, 0)}


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

    if args.workload == "twilight32k":
        return run_twilight(args, dev)
    if args.workload == "offload64k":
        return run_offload(args, dev)
    if args.workload == "tpot32k":
        return run_tpot(args, dev)
    if args.workload == "multireq":
        return run_multireq(args, dev)
    args.context = args.context or 32768
    print(f"[bench] building inputs: layers={args.layers} context={args.context}", file=sys.stderr, flush=True)
    w = QuestWorkload(dev, args.layers, args.context, args.budget_pages, requests=args.requests, union=args.union)

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
    # the split-K kernel alone (phase 1; its partials are merged by phase 2)
    g_att1 = graph_of(lambda: [w.attend(i, phase=1) for i in range(w.layers)])

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
    t_att1 = time_graph(g_att1, reps) / w.layers
    w.step()  # leave a complete step's outputs after the phase-1 replays
    torch.cuda.synchronize()
    by = w.bytes_per_layer()
    layer_bytes = by["select"] + by["attention"]
    layer_s = wall / w.layers
    value = layer_bytes / layer_s / 1e9
    kern = {
        "quest_select": {"us": round(t_sel * 1e6, 2), "bytes": int(by["select"]),
                         "GBps": round(by["select"] / t_sel / 1e9, 1)},
        "decode_attention": {"us": round(t_att1 * 1e6, 2), "bytes": int(by["attention"]),
                             "GBps": round(by["attention"] / t_att1 / 1e9, 1),
                             "kernel": "decode_attn_tiles (split-K, fused decode-token append)"},
        "attention_merge": {"us": round((t_att - t_att1) * 1e6, 2), "kernel": "merge_vec_kernel"},
    }
    # the split-K attention is the longest single kernel of the layer (the
    # selection entry is two launches: score and top-k + union)
    dom = "decode_attention"
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
            "requests": w.requests,
        },
        "layer_us": round(layer_s * 1e6, 3),
        "layer_us_event": round(step_event / w.layers * 1e6, 3),
        "layer_bytes": int(layer_bytes),
        "step_roofline_frac": round(value / HBM_PEAK_GBS, 4),
        "rows_per_group": round(by["rows_per_group"], 1),
        "union_pages_per_group": round(w.union_counts().mean().item(), 1),
        "union_form": w.union,
        "kernels": kern,
        "roofline": {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom), "kernel": dom},
        "parity": parity,
    }
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline + oracle check", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
        parity["oracle"] = result["cpu_baseline"]["oracle_check"]
        parity["ok"] = parity["ok"] and parity["oracle"]["ok"]
    ok = parity["ok"]
    if not args.quest_only:
        # the rest of the metric in the same line: the 4K layer, the Twilight
        # 32K layer (dynamic and matched budgets), the 64K host-offload layer
        # (zero-copy and side-stream DMA), p50 TPOT and the multi-request run
        del w, g_step, g_sel, g_att, g_att1
        torch.cuda.empty_cache()
        leg_args = argparse.Namespace(**vars(args))
        leg_args.steps, leg_args.warmup = 50, 5
        leg_args.cpu_seconds = args.cpu_seconds / 2
        leg_args.context = None
        print("[bench] leg: quest4k", file=sys.stderr, flush=True)
        q4 = quest4k_leg(leg_args, dev)
        result["quest4k"] = q4
        print("[bench] leg: twilight32k", file=sys.stderr, flush=True)
        tw = twilight_leg(leg_args, dev)
        result["twilight32k"] = _leg_summary(tw)
        # the same layer with matched budgets, the reference cache's default budget mode
        print("[bench] leg: twilight32k matched", file=sys.stderr, flush=True)
        m_args = argparse.Namespace(**vars(leg_args))
        m_args.budget_mode, m_args.twilight_path = "matched", "fused"
        twm = twilight_leg(m_args, dev)
        result["twilight32k_matched"] = _leg_summary(twm)
        print("[bench] leg: multireq", file=sys.stderr, flush=True)
        mr = multireq_leg(leg_args, dev)
        result["multireq"] = {k: mr[k] for k in ("value", "unit", "ms_per_step", "layer_us", "hbm_GBps",
                                                 "host_link_GBps", "host_link_frac_pcie_gen5_x16",
                                                 "rows_per_group", "steps")}
        result["multireq"]["contexts"] = mr["config"]["contexts"]
        result["multireq"]["parity_ok"] = mr["parity"]["ok"]
        _release_pinned()
        print("[bench] leg: offload64k", file=sys.stderr, flush=True)
        off_args = argparse.Namespace(**vars(leg_args))
        off_args.no_cpu_baseline = True
        off = offload_leg(off_args, dev)
        result["offload64k"] = {"layer_us": off["layer_us"], "host_link": off["host_link"],
                                "parity_ok": off["parity"]["ok"]}
        _release_pinned()
        print("[bench] leg: tpot32k", file=sys.stderr, flush=True)
        model = tpot_model(dev)
        result["tpot32k"] = tpot_leg(leg_args, dev, model)
        if not args.no_host_tpot:
            print("[bench] leg: tpot64k host", file=sys.stderr, flush=True)
            result["tpot64k_host"] = tpot_leg(leg_args, dev, model, ctx=65536, kv="host", n_dec=16)
        del model
        torch.cuda.empty_cache()
        ok = (ok and q4["parity_ok"] and tw["parity"]["ok"] and twm["parity"]["ok"] and off["parity"]["ok"]
              and mr["parity"]["ok"])
    print(json.dumps(result), flush=True)
    return 0 if ok else 1


def _release_pinned() -> None:
    """Return the pinned host blocks a finished leg freed to the system
    (torch keeps freed pinned memory cached; the next leg's slab is tens of
    GB)."""
    import gc

    import torch

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch._C._host_emptyCache()


def _leg_summary(leg: dict) -> dict:
    out = {k: leg[k] for k in ("layer_us", "kernels", "rows_per_group", "candidate_rows_per_group", "roofline")}
    out["GBps"] = leg["value"]
    out["parity_ok"] = leg["parity"]["ok"]
    if "cpu_baseline" in leg:
        out["cpu_baseline"] = leg["cpu_baseline"]
    return out


def quest4k_leg(args, dev) -> dict:
    """The 4K fp16 layer (8 KV heads x 4 query heads, k = 16 pages, 4 planted
    pages, no outlier channels, seed 0): the configuration the reference's
    torch-CPU path is quoted on, timed on the host cores (the CPU baseline
    and its oracle check) and on the GPU through the same launches as the
    32K layer."""
    import torch

    w = QuestWorkload(dev, args.layers, 4096, 16, seed=0, planted=4, outliers=0)
    w.step()
    torch.cuda.synchronize()
    par = check_parity(w)
    g_step = graph_of(w.step)
    wall, _ = _timed_steps(g_step, args.steps, args.warmup)
    w.step()
    torch.cuda.synchronize()
    by = w.bytes_per_layer()
    layer_s = wall / w.layers
    res = {"layer_us": round(layer_s * 1e6, 3), "GBps": round((by["select"] + by["attention"]) / layer_s / 1e9, 1),
           "context": w.L, "budget_pages": w.k, "scored_pages": w.P, "rows_per_group": round(by["rows_per_group"], 1),
           "dtype": "f16"}
    ok = par["ok"]
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
        ok = ok and res["cpu_baseline"]["oracle_check"]["ok"]
    res["parity_ok"] = ok
    del w, g_step
    torch.cuda.empty_cache()
    return res


def _timed_steps(step_graph, steps: int, warmup: int) -> tuple[float, float]:
    """(wall seconds per replay, event seconds per replay) over `steps`."""
    import torch

    for _ in range(warmup):
        step_graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step_graph.replay()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / max(1, steps)
    return wall, time_graph(step_graph, steps)


def _attention_check(q, keys, vals, rows, masks, cur_k, cur_v, out) -> float:
    """Max abs error of out [R, D] against a float64 recomputation over the
    given rows plus the decode token (None masks: every head sees every row)."""
    import torch

    R, D = q.shape
    kk = torch.cat([keys[rows], cur_k[None]]).double()
    vv = torch.cat([vals[rows], cur_v[None]]).double()
    s = (kk @ q.double().T) / math.sqrt(D)
    if masks is not None:
        m = torch.cat([masks.long(), torch.tensor([(1 << R) - 1], device=masks.device)])
        vis = ((m.unsqueeze(1) >> torch.arange(R, device=m.device)) & 1).bool()
        s = s.masked_fill(~vis, float("-inf"))
    ref = torch.softmax(s, dim=0).T @ vv
    err = (out.double() - ref).abs()
    ok = bool((err <= 2e-3 + 1e-2 * ref.abs()).all().item())
    return float(err.max()) if ok else float("inf")


def run_twilight(args, dev) -> int:
    result = twilight_leg(args, dev)
    print(json.dumps(result), flush=True)
    return 0 if result["parity"]["ok"] else 1


_TW_PATHS = {"fused": "score + per-head B0/INT4 QK/top-p launch (+ the matched allocation launch) into a union "
                      "record, attention over its row masks",
             "pages": "over the B0 union pages row masks", "rows": "over the union row list"}


def twilight_leg(args, dev) -> dict:
    """Twilight at 32K: one decode step of 32 layers x (Quest B0 + INT4 QK +
    top-p + GQA union, then sparse attention over the union and the append)."""
    import torch

    from headinfer import kernels

    ctx = args.context or 32768
    print(f"[bench] twilight inputs: layers={args.layers} context={ctx}", file=sys.stderr, flush=True)
    w = TwilightWorkload(dev, args.layers, ctx, args.budget_mode, path=args.twilight_path)
    w.step()
    torch.cuda.synchronize()
    # structure + attention of layer 0: union ascending, sink and recent present, within bounds
    ok = True
    err = 0.0
    sink_end = min(w.SINK, w.L)
    recent_start = max(sink_end, w.L - (w.RECENT - 1))
    for g in range(w.G):
        rows = w.kept_rows(0, g)
        n = rows.numel()
        ok &= bool((rows[1:] > rows[:-1]).all()) and int(rows[0]) == 0 and int(rows[-1]) == w.L - 1
        ok &= n >= sink_end + (w.L - recent_start) and bool((w.desired[0, g] >= 1).all())
        e = _attention_check(w.q[0, g], w.kc[0, g, : w.L], w.vc[0, g, : w.L], rows, None, w.cur_k[0, g],
                             w.cur_v[0, g], w.out[0, g])
        ok &= e != float("inf")
        err = max(err, e)
    if getattr(args, "calibration_copy", False):
        # a 256 MiB device copy of known size, for scaling the counters of a profiled run
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        torch.empty_like(src).copy_(src)
        torch.cuda.synchronize()
        del src
    g_step = graph_of(w.step)
    g_sel = graph_of(lambda: [w.select(i) for i in range(w.layers)])
    g_att = graph_of(lambda: [w.attend(i) for i in range(w.layers)])
    g_att1 = graph_of(lambda: [w.attend(i, phase=1) for i in range(w.layers)]) if w.fused else None
    # the fused selection's first launch alone (score + INT4 QK of every
    # scored row), for the per-head launch's share of the selection
    g_score = graph_of(lambda: [w.select(i, phase=1) for i in range(w.layers)]) if w.fused else None
    wall, _ = _timed_steps(g_step, args.steps, args.warmup)
    reps = max(20, args.steps // 2)
    t_sel = time_graph(g_sel, reps) / w.layers
    t_att = time_graph(g_att, reps) / w.layers
    t_att1 = time_graph(g_att1, reps) / w.layers if g_att1 is not None else t_att
    t_score = time_graph(g_score, reps) / w.layers if g_score is not None else 0.0
    w.step()  # leave a complete step's outputs after the partial replays
    torch.cuda.synchronize()
    by = w.bytes_per_layer()
    layer_s = wall / w.layers
    value = (by["select"] + by["attention"]) / layer_s / 1e9
    t_head = max(t_sel - t_score, 1e-9)
    kern = {"twilight_select": {"us": round(t_sel * 1e6, 2), "bytes": int(by["select"]),
                                "GBps": round(by["select"] / t_sel / 1e9, 1)},
            "score_qk": {"us": round(t_score * 1e6, 2), "bytes": int(by["score"]),
                         "GBps": round(by["score"] / max(t_score, 1e-9) / 1e9, 1),
                         "kernel": "twilight_score_qk_kernel (Quest score + INT4 QK of every scored row)"},
            "twilight_head": {"us": round(t_head * 1e6, 2), "bytes": int(by["head"]),
                              "GBps": round(by["head"] / t_head / 1e9, 1),
                              "kernel": "twilight_topp_head_kernel" + (" + twilight_matched_rec_kernel"
                                                                       if w.mode == "matched" else ""),
                              "us_from": "selection graph - score + QK graph"},
            "decode_attention": {"us": round(t_att1 * 1e6, 2), "bytes": int(by["attention"]),
                                 "GBps": round(by["attention"] / t_att1 / 1e9, 1),
                                 "kernel": "decode_attn_tiles over the union record (split-K, fused append)"},
            "attention_merge": {"us": round((t_att - t_att1) * 1e6, 2), "kernel": "merge_vec_kernel"}}
    if not w.fused:
        for name in ("score_qk", "twilight_head", "attention_merge"):
            kern.pop(name)
    # the longest single kernel of the layer (with matched budgets the head
    # entry is two launches, the top-p counts and the allocation)
    dom = "decode_attention"
    if w.fused:
        for name in ("score_qk", "twilight_head") if w.mode == "dynamic" else ("score_qk",):
            if kern[name]["us"] > kern[dom]["us"]:
                dom = name
    traffic = (measured_traffic(dom, TWILIGHT_PROFILE if w.mode == "dynamic" else TWILIGHT_MATCHED_PROFILE)
               if w.fused else None)
    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "twilight-32k-hbm: Llama-3-8B-shaped layer x 32, Quest B0 4096 tokens, INT4 QK, "
                               f"top-p {w.TOP_P} ({w.mode} budgets), union attention "
                               f"({_TW_PATHS[w.path]}), "
                               "KV in HBM",
                   "layers": w.layers, "context": w.L, "kv_heads": w.G, "q_per_kv": w.R, "head_dim": w.D,
                   "page_size": w.BS, "b0_pages": w.b0, "top_p": w.TOP_P, "budget_mode": w.mode},
        "layer_us": round(layer_s * 1e6, 3),
        "rows_per_group": round(by["rows_per_group"], 1),
        "candidate_rows_per_group": round(by["candidate_rows_per_group"], 1),
        "kernels": kern,
        "roofline": {"bound": "hbm", "achieved": kern[dom]["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kern[dom]["GBps"] / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": dom},
        "parity": {"ok": ok, "attention_max_abs_err": err},
    }
    if not args.no_cpu_baseline:
        print(f"[bench] twilight {w.mode}: CPU baseline + oracle check", file=sys.stderr, flush=True)
        result["cpu_baseline"] = twilight_cpu_baseline(w, args.cpu_seconds)
        result["parity"]["oracle"] = result["cpu_baseline"]["oracle_check"]
        result["parity"]["ok"] = ok and result["parity"]["oracle"]["ok"]
    del w
    torch.cuda.empty_cache()
    return result


def run_offload(args, dev) -> int:
    result = offload_leg(args, dev)
    print(json.dumps(result), flush=True)
    return 0 if result["parity"]["ok"] else 1


def offload_leg(args, dev) -> dict:
    """64K layer with the KV in pinned host memory: the attention reads the
    selected pages zero-copy over the host link; the side-stream DMA path is
    timed beside it."""
    import torch

    ctx = args.context or 65536
    print(f"[bench] offload inputs: layers={args.layers} context={ctx}", file=sys.stderr, flush=True)
    w = OffloadWorkload(dev, args.layers, ctx, args.budget_pages)
    w.step()
    torch.cuda.synchronize()
    ok = True
    err = 0.0
    sink_end = min(w.SINK, w.L)
    recent_start = max(sink_end, w.L - (w.RECENT - 1))
    for g in range(w.G):
        nu = int(w.plan_counts[0, g])
        pages = w.plan_pages[0, g, :nu].long().cpu()
        pm = w.plan_masks[0, g, :nu].cpu()
        rows = torch.cat([torch.arange(sink_end), (w.SINK + pages[:, None] * w.BS + torch.arange(w.BS)).reshape(-1),
                          torch.arange(recent_start, w.L)])
        masks = torch.cat([torch.full((sink_end,), (1 << w.R) - 1), pm.long().repeat_interleave(w.BS),
                           torch.full((w.L - recent_start,), (1 << w.R) - 1)])
        e = _attention_check(w.q[0, g].cpu(), w.hk[0, g], w.hv[0, g], rows, masks, w.cur_k[0, g].cpu(),
                             w.cur_v[0, g].cpu(), w.out[0, g].cpu())
        ok &= e != float("inf")
        err = max(err, e)
    g_step = graph_of(w.step)
    steps = max(5, args.steps // 10)
    wall, _ = _timed_steps(g_step, steps, min(args.warmup, 5))
    layer_s = wall / w.layers
    host_bytes = w.host_bytes_per_layer()
    by = w.bytes_per_layer()
    # the DMA alternative for comparison: eager (the page ids go to the host
    # once per layer), side-stream copies overlapped with the CPU gather and
    # each group's attention; checked against float64 like the zero-copy path
    w.step()
    torch.cuda.synchronize()
    dma_layers = min(w.layers, 8)
    w.select(0)
    w.attend_dma(0)
    torch.cuda.synchronize()
    for g in range(w.G):
        nu = int(w.plan_counts[0, g])
        pages = w.plan_pages[0, g, :nu].long().cpu()
        pm = w.plan_masks[0, g, :nu].cpu()
        rows = torch.cat([torch.arange(sink_end), (w.SINK + pages[:, None] * w.BS + torch.arange(w.BS)).reshape(-1),
                          torch.arange(recent_start, w.L)])
        masks = torch.cat([torch.full((sink_end,), (1 << w.R) - 1), pm.long().repeat_interleave(w.BS),
                           torch.full((w.L - recent_start,), (1 << w.R) - 1)])
        e = _attention_check(w.q[0, g].cpu(), w.hk[0, g], w.hv[0, g], rows, masks, w.cur_k[0, g].cpu(),
                             w.cur_v[0, g].cpu(), w.out[0, g].cpu())
        ok &= e != float("inf")
        err = max(err, e)
    for layer in range(dma_layers):  # warm: first CPU touch of each layer's slab rows
        w.select(layer)
        w.attend_dma(layer)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for layer in range(dma_layers):
        w.select(layer)
        w.attend_dma(layer)
    torch.cuda.synchronize()
    dma_layer_s = (time.perf_counter() - t0) / dma_layers
    # pinned host -> device copy rate of this box (the host link's practical peak)
    big = torch.empty(1 << 30, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst.copy_(big, non_blocking=True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(3):
        dst.copy_(big, non_blocking=True)
    e1.record()
    torch.cuda.synchronize()
    h2d_gbs = 3 * (1 << 30) / (e0.elapsed_time(e1) / 1e3) / 1e9
    del big, dst
    link = host_bytes / layer_s / 1e9
    result = {
        "metric": METRIC, "value": round((by["select"] + host_bytes) / layer_s / 1e9, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": steps, "warmup": min(args.warmup, 5), "ms_per_step": round(wall * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": "offload-64k-host: Llama-3-8B-shaped layer x 32, KV in pinned host memory, page "
                               "metadata in HBM, Quest selection, attention reading the selected pages zero-copy",
                   "layers": w.layers, "context": w.L, "kv_heads": w.G, "q_per_kv": w.R, "head_dim": w.D,
                   "page_size": w.BS, "budget_pages": w.k},
        "layer_us": round(layer_s * 1e6, 3),
        "host_link": {"bytes_per_layer": int(host_bytes), "zero_copy_GBps": round(link, 2),
                      "pinned_h2d_copy_GBps": round(h2d_gbs, 2), "pcie_gen5_x16_GBps": 64.0,
                      "frac_of_pcie": round(link / 64.0, 4), "frac_of_measured_copy": round(link / h2d_gbs, 4),
                      "dma_path_layer_us": round(dma_layer_s * 1e6, 1),
                      "dma_path_GBps": round(host_bytes / dma_layer_s / 1e9, 2)},
        "rows_per_group": round(host_bytes / (2 * w.D * 2) / w.G, 1),
        "parity": {"ok": ok, "attention_max_abs_err": err},
    }
    del w
    torch.cuda.empty_cache()
    return result


# rocprofv3 FETCH_SIZE / WRITE_SIZE of each kernel, calibrated against a copy
# of known size and recorded with the commands that produced them.
def llama3_8b_config(layers: int = 32):
    """Llama-3-8B shape: hidden 4096, FFN 14336, 32 query / 8 KV heads of 128,
    vocab 128256, RoPE theta 500000."""
    from transformers import LlamaConfig

    return LlamaConfig(hidden_size=4096, intermediate_size=14336, num_hidden_layers=layers, num_attention_heads=32,
                       num_key_value_heads=8, head_dim=128, vocab_size=128256, max_position_embeddings=131072,
                       rope_theta=500000.0, rms_norm_eps=1e-5, tie_word_embeddings=False)


def tpot_run(model, ids, dev, cache, decode_tokens: int, graph: bool = False, dense: bool = False) -> dict:
    """Prefill `ids` into `cache` through the patched model, then decode
    `decode_tokens` tokens of the fixed id 1 -- through the HF forward, or
    (graph) as replays of one captured decode graph (headinfer.graph_decode;
    D1 includes its capture); per-token synchronized wall time, p50 and mean
    over D2..Dn (run_ruler_partial_h2d_tpot_case_v1.py:1302-1322,1897-1906)."""
    import torch

    from headinfer.graph_decode import GraphDecoder

    with torch.no_grad():
        t0 = time.perf_counter()
        model(input_ids=ids.to(dev), past_key_values=cache, use_cache=True, logits_to_keep=1)
        torch.cuda.synchronize()
        prefill_s = time.perf_counter() - t0
        tok = torch.ones((1, 1), dtype=torch.long, device=dev)
        dec = GraphDecoder(model, cache, max_new_tokens=decode_tokens, fixed_token=1,
                           dense=dense) if graph else None
        times = []
        for _ in range(decode_tokens):
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            if dec is not None:
                dec.step()
            else:
                model(input_ids=tok, past_key_values=cache, use_cache=True)
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t1)
    steady = sorted(times[1:]) if len(times) > 1 else times
    return {"tpot_p50_ms": round(steady[len(steady) // 2] * 1e3, 3),
            "tpot_mean_ms": round(sum(steady) / len(steady) * 1e3, 3),
            "d1_ms": round(times[0] * 1e3, 3), "prefill_s": round(prefill_s, 2), "decode_tokens": len(times)}


def run_tpot(args, dev) -> int:
    """End-to-end decode TPOT at 32K context: a Llama-3-8B-shaped model with
    random-init bf16 weights, patched by mp_headinfer, KV in HBM through the
    Quest cache (budget 128 pages = 2048 tokens per query head, sink 64,
    recent 256, page 16).  A random 32K-token prompt is prefilled (dense
    causal attention), then tokens of the fixed id 1 are decoded; TPOT is the
    synchronized wall time per token, p50 over D2..Dn.  The dense comparison
    is the graph decoder with no score or top-k: every whole page before the
    recent window through the same attention kernels."""
    import torch

    from headinfer import mp
    from headinfer.quest_offload_cache import QuestTopKOffloadedCache
    from headinfer.twilight_offload_cache import TwilightMatchedBudgetOffloadedCache
    from transformers import LlamaForCausalLM

    ctx = args.context or 32768
    n_dec = max(2, args.decode_tokens)
    residency = args.kv_residency
    cfg = llama3_8b_config(args.layers)
    print(f"[bench] tpot: Llama-3-8B-shaped x{args.layers} layers, random init, context {ctx}", file=sys.stderr,
          flush=True)
    torch.manual_seed(4)
    with torch.device(dev):
        model = LlamaForCausalLM._from_config(cfg, dtype=torch.bfloat16)
    model.eval()
    mp.mp_headinfer(model)
    ids = torch.randint(0, cfg.vocab_size, (1, ctx), generator=torch.Generator().manual_seed(5))
    runs = {}
    # dense_graph: no score or top-k, every whole page through the same
    # attention; allpages_hf_eager: the HF forward with a budget covering every page
    variants = [("sparse_graph", args.budget_pages, True, False), ("dense_graph", args.budget_pages, True, False),
                ("sparse_hf_eager", args.budget_pages, False, False), ("allpages_hf_eager", 1 << 20, False, False),
                ("twilight_graph", None, True, False), ("twilight_hf_eager", None, False, False)]
    if residency == "host":  # the HBM resident page cache (previous_token_resident_cache) serves host slabs
        variants[1:1] = [("sparse_graph_resident", args.budget_pages, True, True)]
        variants[4:4] = [("sparse_hf_eager_resident", args.budget_pages, False, True)]
        variants.append(("twilight_graph_resident", None, True, True))
        # the reference's own decode path for its resident cache: the HF forward
        # through update_layer_gqa_group_ragged (GQA-group packing + varlen attention)
        variants.append(("twilight_gqa_hf_eager", None, False, False))
        variants.append(("twilight_gqa_hf_eager_resident", None, False, True))
    if args.tpot_only is not None:
        variants = [v for v in variants if v[0] == args.tpot_only]
        if not variants:
            raise SystemExit(f"--tpot-only: no variant named {args.tpot_only!r}")
    for label, pages, graph, resident in variants:
        print(f"[bench] tpot {label}: prefill + {n_dec} decode tokens", file=sys.stderr, flush=True)
        if label.startswith("twilight"):
            # the reference runner's path: Quest B0 = 4096 tokens, INT4 QK, top-p 0.95
            # (resident: with the execution flags the reference requires for its resident cache)
            flags = dict(previous_token_resident_cache=True, layer_batched_selection=True,
                         gqa_groupwise_execution=True, cpu_flat_gather=True, direct_attention_layout=True,
                         gather_h2d_chunks=1) if resident else {}
            if "_gqa_" in label and not resident:
                flags = dict(layer_batched_selection=True, gqa_groupwise_execution=True)
            cache = TwilightMatchedBudgetOffloadedCache.from_llama_model(
                model, max_cache_len=ctx + n_dec + 8, kv_residency=residency, candidate_token_budget=4096,
                top_p=0.95, budget_mode="dynamic", update_metadata_on_decode=graph, **flags)
        else:
            cache = QuestTopKOffloadedCache.from_llama_model(model, max_cache_len=ctx + n_dec + 8,
                                                             kv_residency=residency, budget_pages=pages,
                                                             update_metadata_on_decode=graph,
                                                             previous_token_resident_cache=resident)
        runs[label] = tpot_run(model, ids, dev, cache, n_dec, graph=graph, dense=label == "dense_graph")
        if resident:
            st = cache.resident_stats()
            runs[label]["resident_hit_ratio"] = round(st["resident_hit_pages"] / max(1, st["union_pages"]), 4)
        del cache
        torch.cuda.empty_cache()
    head = "sparse_graph_resident" if residency == "host" else "sparse_graph"
    if head not in runs:
        head = next(iter(runs))
    sp = runs[head]
    result = {
        "metric": METRIC, "value": sp["tpot_p50_ms"], "unit": "ms/token (p50 TPOT)", "n_gpus": 1,
        "steps": n_dec, "warmup": 1, "ms_per_step": sp["tpot_p50_ms"], "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: random-init weights, random prompt ids, fixed decode token id 1",
        "config": {"workload": f"tpot-{ctx // 1024}k-{residency}: Llama-3-8B-shaped decode (HF LlamaForCausalLM "
                               "patched by mp_headinfer), Quest sparse attention, KV in "
                               + ("HBM" if residency == "hbm" else "pinned host memory read zero-copy"),
                   "layers": args.layers, "context": ctx, "kv_heads": 8, "q_per_kv": 4, "head_dim": 128,
                   "page_size": 16, "budget_pages": args.budget_pages, "sink": 64, "recent": 256},
        "tpot_variant": head,
        "tpot": runs,
    }
    if "dense_graph" in runs:
        result["sparse_vs_dense_speedup"] = round(runs["dense_graph"]["tpot_p50_ms"] / sp["tpot_p50_ms"], 3)
    print(json.dumps(result), flush=True)
    return 0


def _graph_tpot(dec, n: int) -> dict:
    """Synchronized wall time of n graph-decoded tokens (D1 includes the
    capture); p50 and mean over D2..Dn (run_ruler_partial_h2d_tpot_case_v1.py:
    1302-1322,1897-1906)."""
    import torch

    times = []
    with torch.no_grad():
        for _ in range(n):
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            dec.step()
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t1)
    steady = sorted(times[1:])
    return {"tpot_p50_ms": round(steady[len(steady) // 2] * 1e3, 3),
            "tpot_mean_ms": round(sum(steady) / len(steady) * 1e3, 3), "decode_tokens": n}


def tpot_model(dev):
    """The Llama-3-8B-shaped model (random-init bf16 weights) patched by
    mp_headinfer, shared by the TPOT legs."""
    import torch

    from headinfer import mp
    from transformers import LlamaForCausalLM

    print("[bench] tpot: Llama-3-8B-shaped model, random init", file=sys.stderr, flush=True)
    torch.manual_seed(4)
    with torch.device(dev):
        model = LlamaForCausalLM._from_config(llama3_8b_config(32), dtype=torch.bfloat16)
    model.eval()
    mp.mp_headinfer(model)
    return model


def tpot_leg(args, dev, model=None, ctx: int = 32768, kv: str = "hbm", n_dec: int = 0) -> dict:
    """p50 TPOT with every decode token one replay of a captured graph: the
    Llama-3-8B-shaped model, a random ctx-token prompt prefilled once per
    cache, then tokens of the fixed id 1.  Decoders: sparse Quest (budget 128
    pages per query head), the dense comparator on the same prefilled cache
    (no score or top-k: every whole page before the recent window through the
    same attention), Twilight (Quest B0 4096 tokens, INT4 QK, top-p 0.95,
    dynamic budgets, then matched budgets on the same cache), and with the KV
    in pinned host memory also sparse Quest and Twilight with the HBM resident
    cache (previous_token_resident_cache)."""
    import torch

    from headinfer.graph_decode import GraphDecoder
    from headinfer.quest_offload_cache import QuestTopKOffloadedCache
    from headinfer.twilight_offload_cache import TwilightMatchedBudgetOffloadedCache

    own = model is None
    if own:
        model = tpot_model(dev)
    n_dec = n_dec or max(4, args.decode_tokens)
    vocab = model.config.vocab_size
    ids = torch.randint(0, vocab, (1, ctx), generator=torch.Generator().manual_seed(5)).to(dev)
    out = {}
    prefill_s = {}

    def prefill(cache, label):
        print(f"[bench] tpot {ctx // 1024}k {kv}: prefill ({label})", file=sys.stderr, flush=True)
        t0 = time.perf_counter()
        model(input_ids=ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
        torch.cuda.synchronize()
        prefill_s[label] = round(time.perf_counter() - t0, 2)

    with torch.no_grad():
        cache = QuestTopKOffloadedCache.from_llama_model(model, max_cache_len=ctx + 2 * n_dec + 8,
                                                         kv_residency=kv, budget_pages=args.budget_pages,
                                                         update_metadata_on_decode=True)
        prefill(cache, "quest")
        dec = GraphDecoder(model, cache, max_new_tokens=n_dec, fixed_token=1)
        out["sparse_graph"] = _graph_tpot(dec, n_dec)
        dec.sync_cache()
        del dec
        dec = GraphDecoder(model, cache, max_new_tokens=n_dec, fixed_token=1, dense=True)
        out["dense_graph"] = _graph_tpot(dec, n_dec)
        del dec, cache
        torch.cuda.empty_cache()
        if kv == "host":
            cache = QuestTopKOffloadedCache.from_llama_model(model, max_cache_len=ctx + n_dec + 8, kv_residency=kv,
                                                             budget_pages=args.budget_pages,
                                                             update_metadata_on_decode=True,
                                                             previous_token_resident_cache=True)
            prefill(cache, "quest, resident page cache")
            dec = GraphDecoder(model, cache, max_new_tokens=n_dec, fixed_token=1)
            out["sparse_graph_resident"] = _graph_tpot(dec, n_dec)
            st = cache.resident_stats()
            out["sparse_graph_resident"]["resident_hit_ratio"] = round(
                st["resident_hit_pages"] / max(1, st["union_pages"]), 4)
            del dec, cache
            torch.cuda.empty_cache()
        cache = TwilightMatchedBudgetOffloadedCache.from_llama_model(
            model, max_cache_len=ctx + 2 * n_dec + 8, kv_residency=kv, candidate_token_budget=4096, top_p=0.95,
            budget_mode="dynamic", update_metadata_on_decode=True)
        prefill(cache, "twilight")
        dec = GraphDecoder(model, cache, max_new_tokens=n_dec, fixed_token=1)
        out["twilight_graph"] = _graph_tpot(dec, n_dec)
        dec.sync_cache()
        del dec
        # the reference cache's default budgets (matched, 5% of the eligible
        # pages), decoding on from the same cache
        cache.budget_mode = "matched"
        dec = GraphDecoder(model, cache, max_new_tokens=n_dec, fixed_token=1)
        out["twilight_matched_graph"] = _graph_tpot(dec, n_dec)
        del dec, cache
        if kv == "host":
            # the Twilight cache's previous-token resident cache (the union rows
            # and the sink/recent windows in HBM), with the execution flags the
            # reference requires for it, on a cache of its own
            torch.cuda.empty_cache()
            cache = TwilightMatchedBudgetOffloadedCache.from_llama_model(
                model, max_cache_len=ctx + n_dec + 8, kv_residency=kv, candidate_token_budget=4096, top_p=0.95,
                budget_mode="dynamic", update_metadata_on_decode=True, previous_token_resident_cache=True,
                layer_batched_selection=True, gqa_groupwise_execution=True, cpu_flat_gather=True,
                direct_attention_layout=True, gather_h2d_chunks=1)
            prefill(cache, "twilight, resident cache")
            dec = GraphDecoder(model, cache, max_new_tokens=n_dec, fixed_token=1)
            out["twilight_graph_resident"] = _graph_tpot(dec, n_dec)
            st = cache.resident_stats()
            out["twilight_graph_resident"]["resident_hit_ratio"] = round(
                st["resident_hit_pages"] / max(1, st["union_pages"]), 4)
            del dec, cache
    if own:
        del model
    torch.cuda.empty_cache()
    dense = out["dense_graph"]["tpot_p50_ms"]
    res = {"context": ctx, "kv": kv, "p50_ms": {k: v["tpot_p50_ms"] for k, v in out.items()},
           "mean_ms": {k: v["tpot_mean_ms"] for k, v in out.items()}, "decode_tokens": n_dec,
           "dense_over": {k: round(dense / v["tpot_p50_ms"], 3) for k, v in out.items() if k != "dense_graph"},
           "prefill_s": prefill_s,
           "model": "Llama-3-8B-shaped (32 layers, 32 q / 8 kv heads, head_dim 128), random-init bf16",
           "budget_pages": args.budget_pages}
    if "sparse_graph_resident" in out:
        res["resident_hit_ratio"] = out["sparse_graph_resident"]["resident_hit_ratio"]
    if "twilight_graph_resident" in out:
        res["twilight_resident_hit_row_ratio"] = out["twilight_graph_resident"]["resident_hit_ratio"]
    return res


class MultiRequestWorkload:
    """Seeded inputs of the multi-request configuration: 8 requests with
    contexts uniform in [16384, 131072] (rounded down to multiples of 16),
    28 layers of a Qwen2.5-7B-like GQA attention (28 query heads, 4 KV heads,
    head_dim 128, bf16), page 16, sink 64, recent 256, Quest budget 128 pages
    per query head.  KV heads {0, 1} of every layer live in HBM, {2, 3} in
    pinned host memory (read zero-copy).  Entries of one residency set are
    ordered (layer, request, head), so a layer's 16 groups are consecutive;
    every group carries its own length in one device array."""

    LAYERS, HQ, HK, D = 28, 28, 4, 128
    R = HQ // HK
    REQUESTS, SINK, RECENT, BS, BUDGET = 8, 64, 256, 16, 128
    STEPS = 256

    def __init__(self, dev, layers: int, seed: int = 4):
        import torch

        from headinfer import kernels

        self.dev, self.layers = dev, layers
        self.kernels = kernels
        g = torch.Generator().manual_seed(seed)
        ctx = torch.randint(16384, 131072 + 1, (self.REQUESTS,), generator=g)
        self.contexts = [int(c) // 16 * 16 for c in ctx]
        self.Lmax = max(self.contexts) + self.STEPS + 16
        self.HS = self.HK // 2                       # KV heads per residency set
        self.G = self.REQUESTS * self.HS             # groups per layer and set
        E = layers * self.G
        self.P = min((self.Lmax - self.SINK) // self.BS, 8192)
        self.width = min(self.P, self.R * self.BUDGET)
        bf = torch.bfloat16
        self.slab = {"hbm": torch.empty((2, E, self.Lmax, self.D), dtype=bf, device=dev),
                     "host": torch.empty((2, E, self.Lmax, self.D), dtype=bf, pin_memory=True)}
        self.pmin = {s: torch.zeros((E, self.P, self.D), dtype=bf, device=dev) for s in self.slab}
        self.pmax = {s: torch.zeros((E, self.P, self.D), dtype=bf, device=dev) for s in self.slab}
        lens = [c for c in self.contexts for _ in range(self.HS)]
        self.lengths = torch.tensor(lens, dtype=torch.int32, device=dev)
        self.lengths0 = list(lens)
        tg = torch.Generator(device=dev).manual_seed(seed + 1)
        for s in self.slab:
            for layer in range(layers):
                e0 = layer * self.G
                kv = torch.randn((2, self.G, self.Lmax, self.D), generator=tg, device=dev, dtype=torch.float32).to(bf)
                for gi, L in enumerate(lens):
                    kernels.build_page_metadata(kv[0, gi, :L], sink=self.SINK, block_size=self.BS,
                                                page_min=self.pmin[s][e0 + gi], page_max=self.pmax[s][e0 + gi])
                self.slab[s][:, e0:e0 + self.G].copy_(kv)
                del kv
        torch.cuda.synchronize()
        self.q = [{s: torch.randn((self.G, self.R, self.D), generator=tg, device=dev).to(bf) for s in self.slab}
                  for _ in range(layers)]
        self.qf = [{s: self.q[i][s].float() for s in self.slab} for i in range(layers)]
        self.cur = [{s: torch.randn((2, self.G, self.D), generator=tg, device=dev).to(bf) for s in self.slab}
                    for _ in range(layers)]
        self.plan = [{s: (torch.zeros((self.G, self.width), dtype=torch.int32, device=dev),
                          torch.zeros((self.G, self.width), dtype=torch.uint8, device=dev),
                          torch.zeros((self.G,), dtype=torch.int32, device=dev)) for s in self.slab}
                     for _ in range(layers)]
        self.out = [{s: torch.empty((self.G, self.R, self.D), dtype=bf, device=dev) for s in self.slab}
                    for _ in range(layers)]

    def layer(self, i: int, s: str) -> None:
        K = self.kernels
        e0 = i * self.G
        pp, pm, pc = self.plan[i][s]
        K.quest_select_ragged(self.qf[i][s], self.pmin[s][e0:e0 + self.G], self.pmax[s][e0:e0 + self.G],
                              self.lengths, self.BUDGET, sink=self.SINK, recent=self.RECENT, block_size=self.BS,
                              plan_pages=pp, plan_masks=pm, plan_counts=pc)
        K.decode_attention_pages_ragged(self.q[i][s], self.slab[s][0, e0:e0 + self.G], self.slab[s][1, e0:e0 + self.G],
                                        pp, pc, self.lengths, plan_masks=pm, max_pages=self.width, sink=self.SINK,
                                        recent=self.RECENT, block_size=self.BS, append=True,
                                        cur_k=self.cur[i][s][0], cur_v=self.cur[i][s][1], out=self.out[i][s])
        K.update_page_metadata_ragged(self.slab[s][0], self.lengths, first_entry=e0, sink=self.SINK,
                                      block_size=self.BS, page_min=self.pmin[s], page_max=self.pmax[s])

    def step(self) -> None:
        for i in range(self.layers):
            for s in ("hbm", "host"):
                self.layer(i, s)
        self.lengths.add_(1)

    def bytes_per_step(self) -> dict:
        """Algorithmic bytes of one step (current plans and lengths): page
        metadata read (2 x D x 2 B per scored page), attended K/V rows
        (2 x D x 2 B), the decode tokens' append; HBM and host link apart."""
        lens = [L - 1 for L in self.lengths.tolist()]  # the lengths the last step ran with
        pages = []
        for L in lens:
            sink_end = min(self.SINK, L)
            recent_start = max(sink_end, L - (self.RECENT - 1))
            pages.append(min(self.P, (recent_start - sink_end) // self.BS))
        row = 2 * self.D * 2
        out = {"hbm": 0.0, "host": 0.0, "rows": {"hbm": 0, "host": 0}}
        for i in range(self.layers):
            for s in ("hbm", "host"):
                counts = self.plan[i][s][2].tolist()
                rows = 0
                for gi, L in enumerate(lens):
                    sink_end = min(self.SINK, L)
                    recent_start = max(sink_end, L - (self.RECENT - 1))
                    rows += sink_end + counts[gi] * self.BS + (L - recent_start)
                out["rows"][s] += rows
                meta = sum(pages) * row
                q_out = 2 * self.G * self.R * self.D * 2
                out["hbm"] += meta + q_out + (rows * row if s == "hbm" else 0) + self.G * row
                if s == "host":
                    out["host"] += rows * row + self.G * row
        return out


def run_multireq(args, dev) -> int:
    result = multireq_leg(args, dev)
    print(json.dumps(result), flush=True)
    return 0 if result["parity"]["ok"] else 1


def multireq_leg(args, dev) -> dict:
    """Multi-request decode: 256 steps of 8 requests x 28 layers, each layer
    one ragged Quest select + one ragged page-tile attention (decode-token
    append fused) + one ragged metadata update per residency set, the step
    captured once as a HIP graph whose replays advance every request's length
    on the device.  1 eager warm-up step, 7 replayed warm-up steps and 248
    timed steps make the 256."""
    import torch

    layers = args.layers if args.layers != 32 else MultiRequestWorkload.LAYERS
    print(f"[bench] multireq inputs: {MultiRequestWorkload.REQUESTS} requests x {layers} layers", file=sys.stderr,
          flush=True)
    t0 = time.perf_counter()
    w = MultiRequestWorkload(dev, layers)
    setup_s = time.perf_counter() - t0
    print(f"[bench] multireq contexts {w.contexts} (setup {setup_s:.1f} s)", file=sys.stderr, flush=True)
    w.step()
    torch.cuda.synchronize()
    g_step = graph_of(w.step, warm=0)
    warm, timed = 7, w.STEPS - 8
    for _ in range(warm):
        g_step.replay()
    torch.cuda.synchronize()
    print(f"[bench] multireq timing {timed} steps", file=sys.stderr, flush=True)
    t1 = time.perf_counter()
    for _ in range(timed):
        g_step.replay()
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t1) / timed
    by = w.bytes_per_step()
    ok, err = multireq_check(w)
    hbm_gbs = by["hbm"] / step_s / 1e9
    host_gbs = by["host"] / step_s / 1e9
    result = {
        "metric": METRIC, "value": round(w.REQUESTS / step_s, 1), "unit": "tokens/s (8 requests, sparse path)",
        "n_gpus": 1, "steps": timed, "warmup": warm + 1, "ms_per_step": round(step_s * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "multireq: Qwen2.5-7B-like GQA (28 q / 4 kv heads, D 128) x 28 layers, 8 requests "
                               "of 16K-128K context, KV heads {0,1} in HBM and {2,3} in pinned host memory, "
                               "256 decode steps with append and page-metadata update, one graph per step",
                   "layers": layers, "requests": w.REQUESTS, "contexts": w.contexts, "q_heads": w.HQ,
                   "kv_heads": w.HK, "head_dim": w.D, "page_size": w.BS, "budget_pages": w.BUDGET,
                   "sink": w.SINK, "recent": w.RECENT, "total_steps": w.STEPS},
        "step_ms": round(step_s * 1e3, 3),
        "layer_us": round(step_s / layers * 1e6, 2),
        "hbm_bytes_per_step": int(by["hbm"]), "host_bytes_per_step": int(by["host"]),
        "hbm_GBps": round(hbm_gbs, 1), "host_link_GBps": round(host_gbs, 2),
        "host_link_frac_pcie_gen5_x16": round(host_gbs / 64.0, 4),
        "rows_per_group": {s: round(by["rows"][s] / (w.G * layers), 1) for s in ("hbm", "host")},
        "setup_s": round(setup_s, 1),
        "parity": {"ok": ok, "attention_max_abs_err": err},
    }
    del w, g_step
    torch.cuda.empty_cache()
    return result


def multireq_check(w) -> tuple[bool, float]:
    """After the run: layer 0's attention of the last step against float64
    over each group's own rows (HBM and host sets, every group), and the
    page metadata of layer 0's entries against a rebuild over their rows."""
    import numpy as np
    import torch

    from headinfer import kernels

    ok, err = True, 0.0
    lens = [L - 1 for L in w.lengths.tolist()]
    for s in ("hbm", "host"):
        pp, pm, pc = (t.cpu() for t in w.plan[0][s])
        kc = w.slab[s][0, :w.G].cpu() if s == "host" else w.slab[s][0, :w.G]
        vc = w.slab[s][1, :w.G].cpu() if s == "host" else w.slab[s][1, :w.G]
        q = w.q[0][s].cpu().double()
        out = w.out[0][s].cpu().double()
        for gi, L in enumerate(lens):
            sink_end = min(w.SINK, L)
            recent_start = max(sink_end, L - (w.RECENT - 1))
            n = int(pc[gi])
            pages = pp[gi, :n].long()
            rows = torch.cat([torch.arange(sink_end), (w.SINK + pages[:, None] * w.BS + torch.arange(w.BS)).reshape(-1),
                              torch.arange(recent_start, L + 1)])  # the decode token was appended at row L
            kk = kc[gi][rows.to(kc.device)].cpu().double()
            vv = vc[gi][rows.to(vc.device)].cpu().double()
            masks = torch.cat([torch.full((sink_end,), 0xff), pm[gi, :n].long().repeat_interleave(w.BS),
                               torch.full((L + 1 - recent_start,), 0xff)])
            for r in range(w.R):
                sc = (kk @ q[gi, r]) / math.sqrt(w.D)
                sc = torch.where(((masks >> r) & 1).bool(), sc, torch.tensor(float("-inf"), dtype=sc.dtype))
                p = torch.softmax(sc, dim=0)
                ref = p @ vv
                e = (out[gi, r] - ref).abs()
                err = max(err, float(e.max()))
                ok &= bool((e <= 2e-3 + 1e-2 * ref.abs()).all())
        # metadata of layer 0's entries == a rebuild over each entry's rows
        for gi, L in enumerate(lens):
            keys = w.slab[s][0, gi, :L + 1].to(w.dev)
            pages = (L + 1 - w.SINK) // w.BS
            bmin = torch.empty((max(pages, 1), w.D), dtype=keys.dtype, device=w.dev)
            bmax = torch.empty_like(bmin)
            kernels.build_page_metadata(keys, sink=w.SINK, block_size=w.BS, page_min=bmin, page_max=bmax)
            ok &= bool(torch.equal(bmin[:pages].view(torch.int16), w.pmin[s][gi, :pages].view(torch.int16)))
            ok &= bool(torch.equal(bmax[:pages].view(torch.int16), w.pmax[s][gi, :pages].view(torch.int16)))
    return ok, err


TRAFFIC_PROFILE = ROOT / "profiles" / "pmc_traffic_quest32k.md"
TWILIGHT_PROFILE = ROOT / "profiles" / "pmc_twilight32k.md"
TWILIGHT_MATCHED_PROFILE = ROOT / "profiles" / "kernel_trace_twilight32k_matched.md"
TRAFFIC_KERNEL = {"decode_attention": "decode_attn_tiles", "quest_select": "quest_score_kernel",
                  "twilight_head": "twilight_topp_head_kernel", "score_qk": "twilight_score_qk_kernel"}


def measured_traffic(kernel: str, profile: Path = TRAFFIC_PROFILE):
    """HBM bytes per launch of the named kernel from a committed PMC summary
    (calibrated FETCH_SIZE + WRITE_SIZE), or None when it is absent."""
    try:
        text = profile.read_text()
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
