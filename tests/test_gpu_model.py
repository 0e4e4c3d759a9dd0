"""mp_headinfer on the GPU: a patched Llama decodes through the offload caches.

With a budget that selects every candidate page (Quest) or keeps every
candidate (Twilight, top_p 1), the sparse path attends the sink window, every
whole page before the recent window and the recent window -- all rows but
the partial page between the last whole page and the recent window
(quest_offload_cache.py:330-346).  The unpatched model attends the same rows
through an explicit 4D mask, so the patched model's logits must match its.
The unpatched model runs on the CPU in float32 with the same bf16-rounded weights (dense attention and its DynamicCache); the patched one
runs in bf16 on the GPU, so the comparison allows bf16 activation rounding.
Each decode entry point of the patch is covered: ``decode_layer`` (Quest and
Twilight), the GQA-group ragged branch, the layer-flat ragged branch and the
per-entry ``update`` branch.  Prompt and decode follow the reference runner:
a random prompt, then decode steps with the fixed token id 1
(run_ruler_partial_h2d_tpot_case_v1.py:1302-1322).
"""

from __future__ import annotations

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

T_PROMPT = 600
DECODE_STEPS = 3


def _say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


def _models(dev, seed=0, q_heads=8):
    from transformers import LlamaConfig, LlamaForCausalLM

    def cfg():
        return LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=q_heads,
                           num_key_value_heads=2, head_dim=128, vocab_size=1000, max_position_embeddings=4096,
                           rope_theta=500000.0)

    torch.manual_seed(seed)
    ref = LlamaForCausalLM(cfg())
    with torch.no_grad():
        for p in ref.parameters():
            p.copy_(p.to(torch.bfloat16).float())
    ref.config._attn_implementation = "eager"
    ref = ref.float().eval()
    gpu = LlamaForCausalLM(cfg())
    gpu.load_state_dict(ref.state_dict())
    gpu = gpu.to(device=dev, dtype=torch.bfloat16).eval()
    return ref, gpu


def _cache(kind, gpu):
    from headinfer.quest_offload_cache import QuestTopKOffloadedCache
    from headinfer.twilight_offload_cache import TwilightMatchedBudgetOffloadedCache

    common = dict(max_cache_len=T_PROMPT + DECODE_STEPS + 2, sink_tokens=64, recent_tokens=256, block_size=16)
    if kind == "quest":
        return QuestTopKOffloadedCache.from_llama_model(gpu, kv_residency="hbm", budget_pages=1000, **common)
    if kind == "quest_host_flat":
        return QuestTopKOffloadedCache.from_llama_model(gpu, kv_residency="host", budget_pages=1000,
                                                        layer_batched_selection=True,
                                                        layer_flat_ragged_execution=True, **common)
    if kind == "quest_per_entry":
        return QuestTopKOffloadedCache.from_llama_model(gpu, kv_residency="hbm", budget_pages=1000,
                                                        per_head_varlen_attention_reference=True, **common)
    twilight = dict(candidate_token_budget=4096, top_p=1.0, budget_mode="dynamic", **common)
    if kind == "twilight":
        return TwilightMatchedBudgetOffloadedCache.from_llama_model(gpu, kv_residency="hbm", **twilight)
    if kind == "twilight_groupwise":
        return TwilightMatchedBudgetOffloadedCache.from_llama_model(
            gpu, kv_residency="host", layer_batched_selection=True, gqa_groupwise_execution=True,
            gpu_compact_gqa_union=True, **twilight)
    raise ValueError(kind)


def _sparse_mask(length: int, sink: int = 64, recent: int = 256, bs: int = 16) -> torch.Tensor:
    """Additive [1, 1, 1, length + 1] mask of the decode token's visible rows
    under a budget covering every candidate page."""
    sink_end = min(sink, length)
    recent_start = max(sink_end, length - max(0, recent - 1))
    cand = (recent_start - sink_end) // bs
    keep = torch.zeros(length + 1, dtype=torch.bool)
    keep[:sink_end] = True
    keep[sink:sink + cand * bs] = True
    keep[recent_start:] = True
    mask = torch.zeros((1, 1, 1, length + 1))
    mask[..., ~keep] = torch.finfo(torch.float32).min
    return mask


def _check(got: torch.Tensor, ref: torch.Tensor, what: str) -> None:
    got = got.float().cpu()
    err = (got - ref).abs().max().item()
    scale = ref.abs().max().item()
    assert err <= 0.03 * scale + 1e-3, f"{what}: max abs err {err:.4f} vs logit scale {scale:.4f}"


@pytest.mark.parametrize("kind", ["quest", "quest_host_flat", "quest_per_entry", "twilight", "twilight_groupwise"])
def test_patched_llama_matches_dense(dev, kind):
    from headinfer import mp

    _say(f"[model] {kind}")
    ref, gpu = _models(dev)
    mp.mp_headinfer(gpu)
    cache = _cache(kind, gpu)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 1000, (1, T_PROMPT), generator=g)
    with torch.no_grad():
        out = gpu(input_ids=ids.to(dev), past_key_values=cache, use_cache=True, logits_to_keep=1)
        r = ref(input_ids=ids, use_cache=True, logits_to_keep=1)
        _check(out.logits[0, -1], r.logits[0, -1], "prefill")
        past = r.past_key_values
        tok = torch.ones((1, 1), dtype=torch.long)
        for step in range(DECODE_STEPS):
            out = gpu(input_ids=tok.to(dev), past_key_values=cache, use_cache=True)
            r = ref(input_ids=tok, past_key_values=past, use_cache=True,
                    attention_mask=_sparse_mask(T_PROMPT + step))
            past = r.past_key_values
            _check(out.logits[0, -1], r.logits[0, -1], f"decode step {step}")
    torch.cuda.synchronize()
    assert cache.get_seq_length() == T_PROMPT + DECODE_STEPS


@pytest.mark.parametrize("residency,resident", [("hbm", False), ("host", False), ("host", True)])
def test_graph_decoder_matches_eager(dev, residency, resident):
    """GraphDecoder (one captured graph per token over the ragged kernels)
    == the eager patched model, token by token, with the same cache policy."""
    from headinfer import mp
    from headinfer.graph_decode import GraphDecoder
    from headinfer.quest_offload_cache import QuestTopKOffloadedCache

    _say(f"[graph decoder] {residency} resident={resident}")
    steps = 6
    _, gpu = _models(dev)
    mp.mp_headinfer(gpu)
    kw = dict(max_cache_len=T_PROMPT + steps + 2, sink_tokens=64, recent_tokens=256, block_size=16,
              kv_residency=residency, budget_pages=8, update_metadata_on_decode=True)
    eager_cache = QuestTopKOffloadedCache.from_llama_model(gpu, **kw)
    graph_cache = QuestTopKOffloadedCache.from_llama_model(gpu, previous_token_resident_cache=resident, **kw)
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, 1000, (1, T_PROMPT), generator=g).to(dev)
    tok = torch.ones((1, 1), dtype=torch.long, device=dev)
    with torch.no_grad():
        gpu(input_ids=ids, past_key_values=eager_cache, use_cache=True, logits_to_keep=1)
        gpu(input_ids=ids, past_key_values=graph_cache, use_cache=True, logits_to_keep=1)
        dec = GraphDecoder(gpu, graph_cache, max_new_tokens=steps, fixed_token=1)
        for step in range(steps):
            ref = gpu(input_ids=tok, past_key_values=eager_cache, use_cache=True).logits[0, -1].float()
            got = dec.step()[0].float()
            torch.cuda.synchronize()
            err = (got - ref).abs().max().item()
            assert err <= 0.02 * ref.abs().max().item() + 1e-3, (step, err)
    dec.sync_cache()
    assert graph_cache.get_seq_length() == eager_cache.get_seq_length() == T_PROMPT + steps
    L = T_PROMPT + steps
    for e in range(graph_cache.geometry.num_entries):
        a = graph_cache._key_cache[e, :L].float().cpu()
        b = eager_cache._key_cache[e, :L].float().cpu()
        assert torch.allclose(a, b, atol=2e-2, rtol=2e-2), e


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_step_ops_match_hf_modules(dev, dtype):
    """The graph decoder's fused element-wise kernels against the HF modules
    they stand for, run on the CPU in the same dtype: RoPE bit for bit;
    residual add + RMSNorm and SiLU * up within one unit in the last place
    (reduction order and exp may differ)."""
    from transformers.models.llama.modeling_llama import LlamaRMSNorm, apply_rotary_pos_emb

    from headinfer import kernels

    g = torch.Generator().manual_seed(7)
    H, Hq, Hk, D, I = 4096, 32, 8, 128, 14336
    # residual add + RMSNorm
    h = (torch.randn((1, H), generator=g) * 3).to(dtype)
    delta = torch.randn((1, H), generator=g).to(dtype)
    norm = LlamaRMSNorm(H, eps=1e-5)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * torch.randn(H, generator=g))
    norm = norm.to(dtype)
    ref_h = h + delta
    with torch.no_grad():
        ref = norm(ref_h)
    hd, out = h.to(dev), torch.empty((1, H), dtype=dtype, device=dev)
    kernels.add_rms_norm(hd, delta.to(dev), norm.weight.to(dev), 1e-5, out)
    torch.cuda.synchronize()
    assert torch.equal(hd.cpu().view(torch.int16), ref_h.view(torch.int16))
    ulp = (out.cpu().view(torch.int16).int() - ref.view(torch.int16).int()).abs()
    assert int(ulp.max()) <= 1 and float((ulp == 0).float().mean()) > 0.95
    # RoPE at a device position
    q = torch.randn((Hq, D), generator=g).to(dtype)
    k = torch.randn((Hk, D), generator=g).to(dtype)
    pos = 777
    inv = 1.0 / (500000.0 ** (torch.arange(0, D, 2).float() / D))
    ang = torch.outer(torch.arange(1024).float(), inv)
    emb = torch.cat([ang, ang], dim=-1)
    cos, sin = emb.cos().to(dtype), emb.sin().to(dtype)
    rq, rk = apply_rotary_pos_emb(q[None, :, None], k[None, :, None], cos[pos:pos + 1][None], sin[pos:pos + 1][None])
    qd, kd = q.to(dev), k.to(dev)
    q32 = torch.empty((Hq, D), dtype=torch.float32, device=dev)
    kernels.rope_qk(qd, kd, cos.to(dev), sin.to(dev), torch.tensor([pos], device=dev), q32)
    torch.cuda.synchronize()
    assert torch.equal(qd.cpu().view(torch.int16), rq[0, :, 0].contiguous().view(torch.int16))
    assert torch.equal(kd.cpu().view(torch.int16), rk[0, :, 0].contiguous().view(torch.int16))
    assert torch.equal(q32.cpu(), rq[0, :, 0].float())
    # one-token GEMV (nn.Linear) against an fp32 matmul of the same operands
    # (x held in registers as 2, 4 or 8 chunks a thread; past 16384 elements the
    # rest staged after the weights' loads)
    for N, Kd, with_bias in ((6144, 4096, True), (4096, 14336, False), (1000, 256, True), (300, 6000, True),
                             (512, 20000, False)):
        W = (torch.randn((N, Kd), generator=g) * 0.02).to(dtype)
        xv = torch.randn((1, Kd), generator=g).to(dtype)
        b = torch.randn(N, generator=g).to(dtype) if with_bias else None
        ref = xv.float() @ W.float().T + (b.float() if b is not None else 0.0)
        y = torch.empty((1, N), dtype=dtype, device=dev)
        kernels.gemv(xv.to(dev), W.to(dev), None if b is None else b.to(dev), y)
        torch.cuda.synchronize()
        err = (y.cpu().float() - ref).abs()
        assert bool((err <= 1e-2 * ref.abs() + 2e-3).all()), (N, Kd, float(err.max()))
    # SiLU * up
    gu = (torch.randn((1, 2 * I), generator=g) * 2).to(dtype)
    ref = torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]
    m = torch.empty((1, I), dtype=dtype, device=dev)
    kernels.silu_mul(gu.to(dev), m)
    torch.cuda.synchronize()
    ulp = (m.cpu().view(torch.int16).int() - ref.view(torch.int16).int()).abs()
    assert int(ulp.max()) <= 1 and float((ulp == 0).float().mean()) > 0.95


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rms_norm_gemv_matches_separate_launches(dev, dtype):
    """The GEMV with the residual add + RMSNorm fused before it and RoPE or
    SiLU * up fused after it: the same bits as add_rms_norm, gemv, rope_qk and
    silu_mul launched one by one, and h_out = the updated residual."""
    from headinfer import kernels

    g = torch.Generator().manual_seed(11)

    def rnd(shape, s=1.0):
        return (torch.randn(shape, generator=g) * s).to(dtype).to(dev)

    D = 128
    pos = torch.tensor([321], device=dev)
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2).float() / D))
    emb = torch.cat([torch.outer(torch.arange(512).float(), inv)] * 2, dim=-1)
    cos, sin = emb.cos().to(dtype).to(dev), emb.sin().to(dtype).to(dev)
    for K, Hq, Hk, I, with_delta, with_bias in ((4096, 8, 2, 1024, True, True), (2048, 4, 4, 8200, False, False),
                                                 (8192, 2, 1, 9000, True, False), (1000, 3, 1, 300, True, True)):
        _say(f"[rms_norm_gemv] {dtype} K={K} Hq={Hq} Hk={Hk} I={I} delta={with_delta} bias={with_bias}")
        h, w_norm = rnd((1, K), 3.0), (1 + 0.1 * torch.randn(K, generator=g)).to(dtype).to(dev)
        delta = rnd((1, K)) if with_delta else None
        Nqkv = (Hq + 2 * Hk) * D
        Wqkv, Wgu = rnd((Nqkv, K), 0.02), rnd((2 * I, K), 0.02)
        bqkv = rnd(Nqkv) if with_bias else None
        bgu = rnd(2 * I) if with_bias else None
        # separate launches
        h_ref = h.clone()
        x = torch.empty_like(h)
        kernels.add_rms_norm(h_ref, delta, w_norm, 1e-5, x)
        qkv_ref = kernels.gemv(x, Wqkv, bqkv, torch.empty((1, Nqkv), dtype=dtype, device=dev))
        q_ref32 = torch.empty((Hq, D), dtype=torch.float32, device=dev)
        kernels.rope_qk(qkv_ref[0, :Hq * D].view(Hq, D), qkv_ref[0, Hq * D:(Hq + Hk) * D].view(Hk, D), cos, sin, pos,
                        q_ref32)
        gu = kernels.gemv(x, Wgu, bgu, torch.empty((1, 2 * I), dtype=dtype, device=dev))
        m_ref = kernels.silu_mul(gu, torch.empty((1, I), dtype=dtype, device=dev))
        Wlm = rnd((17000, K), 0.02)   # wide launch shape
        lm_ref = kernels.gemv(x, Wlm, None, torch.empty((1, 17000), dtype=dtype, device=dev))
        # fused
        h_out = torch.full_like(h, 7.0) if with_delta else None
        qkv = torch.empty((1, Nqkv), dtype=dtype, device=dev)
        q32 = torch.empty((Hq, D), dtype=torch.float32, device=dev)
        kernels.rms_norm_gemv(h, delta, w_norm, 1e-5, h_out, Wqkv, bqkv, qkv, epilogue="rope",
                              rope=(Hq, Hk, cos, sin, pos), q32=q32)
        m = kernels.rms_norm_gemv(h, delta, w_norm, 1e-5, h_out, Wgu, bgu, torch.empty((1, I), dtype=dtype,
                                                                                          device=dev),
                                  epilogue="silu")
        lm = kernels.rms_norm_gemv(h, delta, w_norm, 1e-5, h_out, Wlm, None, torch.empty((1, 17000), dtype=dtype,
                                                                                            device=dev))
        torch.cuda.synchronize()
        assert torch.equal(qkv, qkv_ref) and torch.equal(q32, q_ref32)
        assert torch.equal(m, m_ref) and torch.equal(lm, lm_ref)
        if with_delta:
            assert torch.equal(h_out, h_ref)
    with pytest.raises(ValueError):
        kernels.rms_norm_gemv(h, delta, w_norm, 1e-5, h, Wlm, None, lm)   # h_out aliasing h


def test_graph_decoder_fused_equals_unfused(dev):
    """GraphDecoder with the norms, RoPE and SiLU fused into the GEMVs == the
    same decoder with them as launches of their own, bit for bit (the steps
    cross a page completion, so the fused metadata update is exercised)."""
    from headinfer import mp
    from headinfer.graph_decode import GraphDecoder
    from headinfer.quest_offload_cache import QuestTopKOffloadedCache

    steps = 10
    _, gpu = _models(dev)
    mp.mp_headinfer(gpu)
    kw = dict(max_cache_len=T_PROMPT + steps + 2, sink_tokens=64, recent_tokens=256, block_size=16,
              kv_residency="hbm", budget_pages=8, update_metadata_on_decode=True)
    caches = [QuestTopKOffloadedCache.from_llama_model(gpu, **kw) for _ in range(2)]
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 1000, (1, T_PROMPT), generator=g).to(dev)
    with torch.no_grad():
        for c in caches:
            gpu(input_ids=ids, past_key_values=c, use_cache=True, logits_to_keep=1)
        decs = [GraphDecoder(gpu, caches[0], max_new_tokens=steps, fuse=True),
                GraphDecoder(gpu, caches[1], max_new_tokens=steps, fuse=False)]
        for step in range(steps):
            a = decs[0].step().clone()
            b = decs[1].step().clone()
            torch.cuda.synchronize()
            assert torch.equal(a, b), step
            assert torch.equal(decs[0].token, decs[1].token), step
    assert torch.equal(caches[0]._page_min, caches[1]._page_min)
    assert torch.equal(caches[0]._page_max, caches[1]._page_max)
    n = T_PROMPT + steps   # rows beyond are never written
    assert torch.equal(caches[0]._key_cache[:, :n], caches[1]._key_cache[:, :n])
    assert torch.equal(caches[0]._value_cache[:, :n], caches[1]._value_cache[:, :n])


@pytest.mark.parametrize("fuse,mode,q_heads,resident", [(True, "dynamic", 8, False), (False, "dynamic", 8, False),
                                                        (True, "matched", 8, False), (True, "dynamic", 32, False),
                                                        (True, "matched", 32, False), (True, "dynamic", 8, True)])
def test_graph_decoder_twilight_matches_eager(dev, fuse, mode, q_heads, resident):
    """GraphDecoder over a Twilight cache (Quest B0, INT4 QK, top-p and the
    GQA union from device-side lengths, the union attention with the append,
    the INT4 + page metadata update) == the eager patched model with the same
    cache policy, token by token; the steps cross a page completion.  32
    query heads over 2 KV heads (16 per group) run the fused selection and
    the union attention as sub-groups of 8 (matched: one allocation over the
    16 heads).  resident: both caches over a host slab, the graph's with the
    previous-token resident cache (the union rows and windows in HBM)."""
    from headinfer import mp
    from headinfer.graph_decode import GraphDecoder
    from headinfer.twilight_offload_cache import TwilightMatchedBudgetOffloadedCache

    _say(f"[graph decoder twilight] fuse={fuse} {mode} q_heads={q_heads} resident={resident}")
    steps = 10
    _, gpu = _models(dev, q_heads=q_heads)
    mp.mp_headinfer(gpu)
    kw = dict(max_cache_len=T_PROMPT + steps + 2, sink_tokens=64, recent_tokens=256, block_size=16,
              kv_residency="hbm", candidate_token_budget=128, top_p=0.9, budget_mode=mode,
              update_metadata_on_decode=True)
    if resident:
        kw["kv_residency"] = "host"
    eager_cache = TwilightMatchedBudgetOffloadedCache.from_llama_model(gpu, **kw)
    flags = dict(previous_token_resident_cache=True, layer_batched_selection=True, gqa_groupwise_execution=True,
                 cpu_flat_gather=True, direct_attention_layout=True, gather_h2d_chunks=1) if resident else {}
    graph_cache = TwilightMatchedBudgetOffloadedCache.from_llama_model(gpu, **kw, **flags)
    assert graph_cache._resident_active == resident
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(0, 1000, (1, T_PROMPT), generator=g).to(dev)
    tok = torch.ones((1, 1), dtype=torch.long, device=dev)
    with torch.no_grad():
        gpu(input_ids=ids, past_key_values=eager_cache, use_cache=True, logits_to_keep=1)
        gpu(input_ids=ids, past_key_values=graph_cache, use_cache=True, logits_to_keep=1)
        dec = GraphDecoder(gpu, graph_cache, max_new_tokens=steps, fixed_token=1, fuse=fuse)
        for step in range(steps):
            ref = gpu(input_ids=tok, past_key_values=eager_cache, use_cache=True).logits[0, -1].float()
            got = dec.step()[0].float()
            torch.cuda.synchronize()
            err = (got - ref).abs().max().item()
            assert err <= 0.02 * ref.abs().max().item() + 1e-3, (step, err)
    dec.sync_cache()
    L = T_PROMPT + steps
    assert graph_cache.get_seq_length() == eager_cache.get_seq_length() == L
    for e in range(graph_cache.geometry.num_entries):
        a = graph_cache._key_cache[e, :L].float().cpu()
        b = eager_cache._key_cache[e, :L].float().cpu()
        assert torch.allclose(a, b, atol=2e-2, rtol=2e-2), e


def test_graph_decoder_dense_equals_all_pages_budget(dev):
    """The dense comparator (no score or top-k, every page through the page-tile
    attention) == the sparse decoder whose budget covers every page, bit for
    bit: same rows, same tile order, same kernels after the selection."""
    from headinfer import mp
    from headinfer.graph_decode import GraphDecoder
    from headinfer.quest_offload_cache import QuestTopKOffloadedCache

    steps = 6
    _, gpu = _models(dev)
    mp.mp_headinfer(gpu)
    kw = dict(max_cache_len=T_PROMPT + steps + 2, sink_tokens=64, recent_tokens=256, block_size=16,
              kv_residency="hbm", update_metadata_on_decode=True)
    caches = [QuestTopKOffloadedCache.from_llama_model(gpu, budget_pages=1000, **kw),
              QuestTopKOffloadedCache.from_llama_model(gpu, **kw)]
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(0, 1000, (1, T_PROMPT), generator=g).to(dev)
    with torch.no_grad():
        for c in caches:
            gpu(input_ids=ids, past_key_values=c, use_cache=True, logits_to_keep=1)
        decs = [GraphDecoder(gpu, caches[0], max_new_tokens=steps),
                GraphDecoder(gpu, caches[1], max_new_tokens=steps, dense=True)]
        for step in range(steps):
            a = decs[0].step().clone()
            b = decs[1].step().clone()
            torch.cuda.synchronize()
            assert torch.equal(a, b), step
    n = T_PROMPT + steps
    assert torch.equal(caches[0]._key_cache[:, :n], caches[1]._key_cache[:, :n])
