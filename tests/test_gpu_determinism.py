"""Run-to-run determinism of the GPU paths.  Every reduction in the kernels runs in a fixed order
(split-K partials summed in split order, per-chapter sums in the plan's order, no atomics), so two
identical forward + backward calls give bit-identical outputs and gradients.  Covered at the
paper's widths (d = 768, 12 heads, 64-row chapters): the native sequence layer (router, chapter
plan, K/V projection and its dX / dW GEMMs, attention forward, dQ with the fused pre-pass, dK/dV,
the three-stream schedule) and the token-routed layer (token router, whole-bank projection GEMMs,
sparse forward / backward, slot combines) in its v4 (weighted) and joint forms."""

import pytest
import torch

from helpers import gen

pytestmark = pytest.mark.gpu


def _run(dev, kind, weighted, inputs):
    from memory_amd.model import RoutedMemoryLayer, TokenRoutedMemoryLayer
    h, bank, Wr, Wq, Wk, Wv, Wo, dO, shape = inputs
    d, H, C, T, k = shape
    if kind == "sequence":
        layer = RoutedMemoryLayer(d, H, C, T, k, num_shared_chapters=1, routed_scaling_factor=2.5,
                                  wo_init_zero=False)
    else:
        layer = TokenRoutedMemoryLayer(d, H, C, T, k, num_shared_chapters=1, routed_scaling_factor=2.5,
                                       weighted=weighted, wo_init_zero=False)
    with torch.no_grad():
        layer.router.router.weight.copy_(Wr)
        layer.router.router.bias.zero_()
        for lin, W in zip((layer.memory_attn.q_proj, layer.memory_attn.k_proj, layer.memory_attn.v_proj,
                           layer.memory_attn.o_proj), (Wq, Wk, Wv, Wo)):
            lin.weight.copy_(W)
    layer = layer.to(dev)
    for m in (layer.memory_attn.q_proj, layer.memory_attn.k_proj, layer.memory_attn.v_proj, layer.memory_attn.o_proj):
        m.to(torch.bfloat16)
    hg = h.to(dev, torch.bfloat16).requires_grad_(True)
    bg = bank.to(dev, torch.bfloat16).requires_grad_(True)
    out, _ = layer(hg, bg, return_losses=False)
    (out.float() * dO.to(dev)).sum().backward()
    torch.cuda.synchronize()
    named = {"out": out.detach(), "dh": hg.grad, "dbank": bg.grad}
    for n, p in layer.named_parameters():
        if p.grad is not None:
            named["d" + n] = p.grad
    return {n: t.detach().clone() for n, t in named.items()}


@pytest.mark.parametrize("kind,weighted,B,L,C,k", [
    ("sequence", False, 4, 512, 257, 16),
    ("token", True, 2, 256, 129, 8),
    ("token", False, 2, 256, 129, 8),
])
def test_layer_bitwise_repeatable(gpu_device, kind, weighted, B, L, C, k):
    print(f"determinism {kind} weighted={weighted} B={B} L={L} C={C} k={k}", flush=True)
    d, H, T = 768, 12, 64
    g = gen(900 + B + L + C)
    h = torch.randn(B, L, d, generator=g)
    bank = torch.randn(C * T, d, generator=g) * 0.5
    Wr = torch.randn(C, d, generator=g) * 0.05
    Wq, Wk, Wv, Wo = (torch.randn(d, d, generator=g) / d ** 0.5 for _ in range(4))
    dO = torch.randn(B, L, d, generator=g)
    inputs = (h, bank, Wr, Wq, Wk, Wv, Wo, dO, (d, H, C, T, k))
    first = _run(gpu_device, kind, weighted, inputs)
    second = _run(gpu_device, kind, weighted, inputs)
    assert first.keys() == second.keys()
    assert {"out", "dh", "dbank"} <= first.keys()
    for n in first:
        same = torch.equal(first[n], second[n])
        if not same:
            diff = (first[n].float() - second[n].float()).abs().max().item()
            print(f"  {n}: max |run 1 - run 2| = {diff:.3e}", flush=True)
        assert same, n
