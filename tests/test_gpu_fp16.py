"""float16 modules (memory_amd._half): the layers with float16 inputs, bank and parameters run
on the float32 kernels and return float16; outputs and every gradient against the oracle's
float64 layers on the same float16-rounded tensors.  The float16 results carry one rounding of a
float32 computation: the gate is the bfloat16 form (max |a - b| after the exact power-of-two
scaling, and max |a - b| / max |b|) at 2e-3, twice float16's unit roundoff."""

import pytest
import torch

import oracle as O
from helpers import assert_parity, gen

pytestmark = pytest.mark.gpu

H16 = torch.float16
F16_ATOL = 2e-3


def _copy(layer, Wr, br, Wq, Wk, Wv, Wo):
    with torch.no_grad():
        layer.router.router.weight.copy_(Wr)
        layer.router.router.bias.copy_(br)
        for lin, W in zip((layer.memory_attn.q_proj, layer.memory_attn.k_proj, layer.memory_attn.v_proj,
                           layer.memory_attn.o_proj), (Wq, Wk, Wv, Wo)):
            lin.weight.copy_(W)


@pytest.mark.parametrize("kind", ["sequence", "token"])
def test_float16_layers_match_oracle(gpu_device, kind):
    print(f"float16 layer {kind}", flush=True)
    from memory_amd.model import RoutedMemoryLayer, TokenRoutedMemoryLayer
    dev = gpu_device
    g = gen(401)
    B, Lq, d, H, C, T, S, k = 2, 64, 128, 2, 9, 64, 1, 3
    h = torch.randn(B, Lq, d, generator=g).to(H16)
    bank = (torch.randn(C * T, d, generator=g) * 0.5).to(H16)
    Wr = (torch.randn(C, d, generator=g) * 0.3).to(H16)
    br = torch.zeros(C).to(H16)
    Wq, Wk, Wv, Wo = ((torch.randn(d, d, generator=g) / d ** 0.5).to(H16) for _ in range(4))
    if kind == "sequence":
        layer = RoutedMemoryLayer(d, H, C, T, k, num_shared_chapters=S, routed_scaling_factor=2.5, wo_init_zero=False)
    else:
        layer = TokenRoutedMemoryLayer(d, H, C, T, k, num_shared_chapters=S, routed_scaling_factor=2.5,
                                       weighted=False, wo_init_zero=False)
    layer = layer.to(dev).half()
    _copy(layer, Wr, br, Wq, Wk, Wv, Wo)
    hg = h.to(dev).requires_grad_(True)
    bg = bank.to(dev).requires_grad_(True)
    out, _ = layer(hg, bg, return_losses=False)
    assert out.dtype == H16
    dO = torch.randn(out.shape, generator=gen(402))
    (out.float() * dO.to(dev)).sum().backward()
    leaves = [t.double().clone().requires_grad_(True) for t in (h, bank, Wr, br, Wq, Wk, Wv, Wo)]
    if kind == "sequence":
        ref = O.sequence_memory_layer(*leaves, H=H, HK=H, C=C, T=T, S=S, top_k=k, routed_scale=2.5)
    else:
        ref = O.token_memory_layer(*leaves, H=H, HK=H, C=C, T=T, S=S, top_k=k, routed_scale=2.5, weighted=False)
    (ref * dO.double()).sum().backward()
    assert_parity(out, ref, H16, "out", bf16_atol=F16_ATOL)
    got = [hg.grad, bg.grad, layer.router.router.weight.grad, layer.router.router.bias.grad,
           layer.memory_attn.q_proj.weight.grad, layer.memory_attn.k_proj.weight.grad,
           layer.memory_attn.v_proj.weight.grad, layer.memory_attn.o_proj.weight.grad]
    for n, gr, r in zip(["dh", "dbank", "dWr", "dbr", "dWq", "dWk", "dWv", "dWo"], got, leaves):
        if r.grad is None or (kind == "token" and n in ("dWr", "dbr")):
            continue
        assert gr.dtype == H16, n
        assert_parity(gr, r.grad, H16, n, bf16_atol=F16_ATOL)


def test_float16_cross_attention_over_memory(gpu_device):
    """MemoryCrossAttention(hidden, memory) in float16 against the oracle's dense cross-attention."""
    print("float16 cross-attention", flush=True)
    from memory_amd.memory_attention import MemoryCrossAttention
    dev = gpu_device
    g = gen(403)
    B, Lq, N, d, H = 2, 40, 128, 128, 2
    h = torch.randn(B, Lq, d, generator=g).to(H16)
    mem = torch.randn(B, N, d, generator=g).to(H16)
    Ws = [(torch.randn(d, d, generator=g) / d ** 0.5).to(H16) for _ in range(4)]
    m = MemoryCrossAttention(d, H, wo_init_zero=False).to(dev).half()
    with torch.no_grad():
        for lin, W in zip((m.q_proj, m.k_proj, m.v_proj, m.o_proj), Ws):
            lin.weight.copy_(W)
    hg = h.to(dev).requires_grad_(True)
    mg = mem.to(dev).requires_grad_(True)
    out, _ = m(hg, mg)
    assert out.dtype == H16
    dO = torch.randn(out.shape, generator=gen(404))
    (out.float() * dO.to(dev)).sum().backward()
    leaves = [t.double().clone().requires_grad_(True) for t in (h, mem, *Ws)]
    ref = O.cross_attention(leaves[0], leaves[1], *leaves[2:], H, H)
    (ref * dO.double()).sum().backward()
    assert_parity(out, ref, H16, "out", bf16_atol=F16_ATOL)
    for n, gr, r in zip(["dh", "dmemory", "dWq", "dWk", "dWv", "dWo"],
                        [hg.grad, mg.grad, m.q_proj.weight.grad, m.k_proj.weight.grad, m.v_proj.weight.grad,
                         m.o_proj.weight.grad], leaves):
        assert_parity(gr, r.grad, H16, n, bf16_atol=F16_ATOL)
