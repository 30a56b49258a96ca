"""GPU parity of decode-time re-routing (memory_amd.decode.DecodeRouter: the inference
strategies of MemoryTransformer.forward, memory_transformer/model.py:609-661) against the
oracle's ``inference_route``, over a prefill and several generated tokens: router logits within
the fp32 gate, chapter ids bit-exact (selected from the same logits), omega within the fp32 gate,
and every step's decode output against the oracle's decode step on those chapters."""

import pytest
import torch

import oracle as O
from helpers import assert_parity, gen

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("strategy,masked", [("sequence", False), ("sequence-rolling", False), ("rolling", False),
                                             ("hybrid", False), ("rolling", True), ("hybrid", True)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_router_matches_oracle(gpu_device, strategy, masked, dtype):
    print(f"decode routing strategy={strategy} masked={masked} dtype={dtype}", flush=True)
    from memory_amd.decode import DecodeRouter, MemoryDecodeCache, memory_decode_step
    from memory_amd.memory_attention import MemoryCrossAttention
    from memory_amd.router import ChapterRouter
    dev = gpu_device
    g = gen(7 + len(strategy) + 2 * masked)
    B, H, HK, C, k, S, T, P, W, steps = 5, 2, 2, 24, 4, 1, 64, 9, 6, 4
    d = H * 64
    bank = torch.randn(C * T, d, generator=g)
    Wq, Wo = (torch.randn(d, d, generator=g) / d ** 0.5 for _ in range(2))
    Wk, Wv = (torch.randn(HK * 64, d, generator=g) / d ** 0.5 for _ in range(2))
    Wr = torch.randn(C, d, generator=g)
    br = torch.randn(C, generator=g) * 0.5
    attn = MemoryCrossAttention(d, H, HK, wo_init_zero=False)
    router = ChapterRouter(d, C, k)
    with torch.no_grad():
        for lin, Wt in ((attn.q_proj, Wq), (attn.k_proj, Wk), (attn.v_proj, Wv), (attn.o_proj, Wo)):
            lin.weight.copy_(Wt)
        router.router.weight.copy_(Wr)
        router.router.bias.copy_(br)
    attn = attn.to(dev, dtype)
    router = router.to(dev)
    cache = MemoryDecodeCache(bank.to(dev, dtype), attn.k_proj.weight, attn.v_proj.weight, num_chapters=C,
                              tokens_per_chapter=T, num_kv_heads=HK, dtype=dtype)
    dr = DecodeRouter(router, num_chapters=C, num_shared_chapters=S, routed_scaling_factor=2.5, strategy=strategy,
                      window_size=W)
    rd = lambda t: t.to(dtype).double()
    prompt = torch.randn(B, P, d, generator=g)
    mask = None
    if masked:   # left padding of two sequences
        mask = torch.ones(B, P, dtype=torch.long)
        mask[1, :3] = 0
        mask[3, :P - 1] = 0
    ocache = None
    for step in range(steps + 1):
        h = prompt if step == 0 else torch.randn(B, 1, d, generator=g)
        if mask is not None and step > 0:
            mask = torch.cat([mask, torch.ones(B, 1, dtype=torch.long)], dim=1)
        hm = None if mask is None else mask.to(dev)
        routing = dr.prefill(h.to(dev, dtype), hm) if step == 0 else dr.step(h.to(dev, dtype), hm)
        got_logits = dr.last_logits.double().cpu()
        _, ologits, oci, ocw, ocache = O.inference_route(
            strategy, rd(h), ocache, Wr.double(), br.double(), top_k=k, num_shared=S, num_chapters=C,
            routed_scale=2.5, window=W, mask=mask, prefill=step == 0, select_by_logits=got_logits)
        assert_parity(dr.last_logits, ologits, torch.float32, f"step {step} router logits")
        assert torch.equal(routing.idx.long().cpu(), oci), f"step {step}: chapter ids"
        assert_parity(routing.omega, ocw, torch.float32, f"step {step} omega")
        # the step's decode on the chapters just chosen (the last token's hidden states)
        h_t = h[:, -1:]
        out = memory_decode_step(attn, h_t.to(dev, dtype), cache, routing)
        ref = O.decode_step(rd(h_t), rd(bank), oci, ocw, rd(Wq), rd(Wk), rd(Wv), rd(Wo), H=H, HK=HK, T=T, S=S)
        assert_parity(out, ref, dtype, f"step {step} decode output")


def test_dynamic_routing_plan_matches_synced(gpu_device):
    """A routing built without the host read of the distinct-chapter count (launches sized for
    min(B * NS, C) chapters) gives the decode output of the synced one bit for bit."""
    from memory_amd.decode import DecodeRouting, MemoryDecodeCache, memory_decode_step
    from memory_amd.memory_attention import MemoryCrossAttention
    dev = gpu_device
    g = gen(55)
    B, H, HK, C, k, T = 16, 2, 1, 40, 6, 64
    d = H * 64
    attn = MemoryCrossAttention(d, H, HK, wo_init_zero=False).to(dev, torch.bfloat16)
    bank = torch.randn(C * T, d, generator=g).to(dev, torch.bfloat16)
    cache = MemoryDecodeCache(bank, attn.k_proj.weight, attn.v_proj.weight, num_chapters=C, tokens_per_chapter=T,
                              num_kv_heads=HK)
    idx, w, _ = O.route_sequence(torch.randn(B, C, generator=g), k, 1)
    ci, cw = O.prepend_shared_chapters(idx, w, num_chapters=C, num_shared_chapters=1, routed_scaling_factor=2.5)
    h = torch.randn(B, 1, d, generator=g).to(dev, torch.bfloat16)
    synced = DecodeRouting(ci.to(dev), cw.to(dev), C)
    dynamic = DecodeRouting(ci.to(dev), cw.to(dev), C, sync=False)
    assert dynamic.max_units == min(B * (k + 1), C) >= synced.max_units
    assert dynamic.unique_chapters() == synced.unique_chapters() == int(torch.unique(ci).numel())
    a = memory_decode_step(attn, h, cache, synced)
    b = memory_decode_step(attn, h, cache, dynamic)
    assert torch.equal(a, b)
