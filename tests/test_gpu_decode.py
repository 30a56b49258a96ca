"""GPU parity of the decode step (BASELINE config 5 path) against the oracle's
decode_step (the L = 1 case of the sequence-routed layer with fixed chapters
and omega), for fp32 (1e-4) and bf16 (2e-2), with GQA, row normalisation and
chapters shared by many sequences (the shared chapter by all of them)."""

import pytest
import torch

import oracle as O
from helpers import assert_parity, gen

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,H,HK,C,k,norm", [(6, 2, 2, 12, 4, None), (5, 4, 2, 9, 3, "rms"), (64, 2, 2, 65, 16, None),
                                             (3, 2, 1, 7, 6, "layernorm")])
def test_decode_step_matches_oracle(gpu_device, dtype, B, H, HK, C, k, norm):
    print(f"decode dtype={dtype} B={B} H={H} HK={HK} C={C} k={k} norm={norm}", flush=True)
    from memory_amd.decode import DecodeRouting, MemoryDecodeCache, memory_decode_step
    from memory_amd.memory_attention import MemoryCrossAttention
    dev = gpu_device
    g = gen(90 + B + C)
    d, T, S = H * 64, 64, 1
    h = torch.randn(B, 1, d, generator=g)
    bank = torch.randn(C * T, d, generator=g)
    Wq = torch.randn(d, d, generator=g) / d ** 0.5
    Wk = torch.randn(HK * 64, d, generator=g) / d ** 0.5
    Wv = torch.randn(HK * 64, d, generator=g) / d ** 0.5
    Wo = torch.randn(d, d, generator=g) / d ** 0.5
    logits = torch.randn(B, C, generator=g) * 2
    idx, w, _ = O.route_sequence(logits, k, S)
    ci, cw = O.prepend_shared_chapters(idx, w, num_chapters=C, num_shared_chapters=S, routed_scaling_factor=2.5)

    attn = MemoryCrossAttention(d, H, HK, wo_init_zero=False)
    with torch.no_grad():
        for lin, W in ((attn.q_proj, Wq), (attn.k_proj, Wk), (attn.v_proj, Wv), (attn.o_proj, Wo)):
            lin.weight.copy_(W)
    attn = attn.to(dev, dtype)
    cache = MemoryDecodeCache(bank.to(dev, dtype), attn.k_proj.weight, attn.v_proj.weight, num_chapters=C,
                              tokens_per_chapter=T, num_kv_heads=HK, norm_type=norm, eps=1e-5, dtype=dtype)
    routing = DecodeRouting(ci.to(dev), cw.to(dev), C)
    assert routing.unique_chapters() == int(torch.unique(ci).numel())
    out = memory_decode_step(attn, h.to(dev, dtype), cache, routing)

    rd = lambda t: t.to(dtype).double()
    ref = O.decode_step(rd(h), rd(bank), ci, cw.double(), rd(Wq), rd(Wk), rd(Wv), rd(Wo), H=H, HK=HK, T=T,
                        normalize=norm is not None, norm_type=norm or "rms", eps=1e-5, S=S)
    assert_parity(out, ref, dtype, "decode output")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_step_graph_replays_match_eager(gpu_device, dtype):
    """Two memory layers' decode captured as one HIP graph: every replay (with new inputs,
    eager work and synchronisations between replays) equals the eager decode step bit for bit."""
    print(f"decode graph replays dtype={dtype}", flush=True)
    from memory_amd.decode import DecodeRouting, DecodeStepGraph, MemoryDecodeCache, memory_decode_step
    from memory_amd.memory_attention import MemoryCrossAttention
    dev = gpu_device
    g = gen(321)
    B, H, HK, C, k, d, T = 8, 2, 2, 17, 5, 128, 64
    layers = []
    for _ in range(2):
        attn = MemoryCrossAttention(d, H, HK, wo_init_zero=False).to(dev, dtype)
        bank = torch.randn(C * T, d, generator=g).to(dev, dtype)
        cache = MemoryDecodeCache(bank, attn.k_proj.weight, attn.v_proj.weight, num_chapters=C, tokens_per_chapter=T,
                                  num_kv_heads=HK, dtype=dtype)
        idx, w, _ = O.route_sequence(torch.randn(B, C, generator=g), k, 1)
        ci, cw = O.prepend_shared_chapters(idx, w, num_chapters=C, num_shared_chapters=1, routed_scaling_factor=2.5)
        layers.append((attn, cache, DecodeRouting(ci.to(dev), cw.to(dev), C)))
    xs = [torch.randn(B, 1, d, generator=g).to(dev, dtype) for _ in range(2)]
    graph = DecodeStepGraph(layers, xs)
    for rep in range(4):
        inputs = [torch.randn(B, 1, d, generator=g).to(dev, dtype) for _ in range(2)]
        outs = [o.clone() for o in graph.run(inputs)]
        junk = torch.randn(1000, device=dev).sum()          # eager work between replays
        torch.cuda.synchronize()
        ref = [memory_decode_step(a, x, c, r) for (a, c, r), x in zip(layers, inputs)]
        for i, (o, r) in enumerate(zip(outs, ref)):
            assert torch.equal(o, r), f"replay {rep}, layer {i}"
        del junk
    # hidden states written straight into the captured input buffers: replayed without copies
    for rep in range(2):
        for buf in graph.static_in:
            buf.copy_(torch.randn(B, 1, d, generator=g).to(dev, dtype))
        outs = [o.clone() for o in graph.run(graph.static_in)]
        torch.cuda.synchronize()
        ref = [memory_decode_step(a, x.clone(), c, r) for (a, c, r), x in zip(layers, graph.static_in)]
        for i, (o, r) in enumerate(zip(outs, ref)):
            assert torch.equal(o, r), f"in-place replay {rep}, layer {i}"
