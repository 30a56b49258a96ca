"""Parity at the full BASELINE sizes (the shapes bench.py measures), bf16 on the GPU against
the oracle in fp32 on the CPU.

config 3 (B=8, L=1024, d=768, 12 heads, bank 4,097 x 64, S=1 shared + k=64 routed, scale 2.5):
  * routing: each sequence's 64 routed chapters are distinct and form a top-64 of the oracle's
    fp64 router logits up to a tie band of 1e-5 (the GPU logits are fp32 sums, so chapters whose
    logits differ by less than fp32 rounding may swap);
  * output and every gradient (h, bank, q/k/v/o projections, router weight and bias): the
    oracle's gather -> x omega -> cross-attention chain (model.py:677-692,
    memory_attention.py:402-478) evaluated on the GPU's own chapter choice, with omega from the
    oracle's renormalised router probabilities (router.py:114-149, model.py:356-391), so the
    comparison cannot hinge on a near-tie.
config 5 (decode, B=64, k=64, 12 heads over the 4,097-chapter bank): the decode step against
  the oracle's decode_step on the same routing.

Gate (tests/helpers.py): bf16 max-abs 2e-2 on every output and gradient, router weight and
bias gradients included, plus max|a-b|/max|b| <= 2e-2."""

import pytest
import torch

import oracle as O
from helpers import assert_parity

pytestmark = pytest.mark.gpu

B, L, D, H, C, T, S, K, SCALE = 8, 1024, 768, 12, 4097, 64, 1, 64, 2.5


def _config3_check(dev, h, bank, Wr, br, Wq, Wk, Wv, Wo, dO):
    """Run the layer at config 3 on the GPU and check routing, output and every gradient
    against the oracle chain on the GPU's chapter choice (all tensors on the CPU, bf16 where
    the GPU holds bf16, fp32 router weights)."""
    from memory_amd.model import RoutedMemoryLayer
    bf = torch.bfloat16
    layer = RoutedMemoryLayer(D, H, C, T, K, num_shared_chapters=S, routed_scaling_factor=SCALE,
                              wo_init_zero=False)
    with torch.no_grad():
        layer.router.router.weight.copy_(Wr)
        layer.router.router.bias.copy_(br)
        for lin, W in ((layer.memory_attn.q_proj, Wq), (layer.memory_attn.k_proj, Wk),
                       (layer.memory_attn.v_proj, Wv), (layer.memory_attn.o_proj, Wo)):
            lin.weight.copy_(W.float())
    layer = layer.to(dev)
    for m in (layer.memory_attn.q_proj, layer.memory_attn.k_proj, layer.memory_attn.v_proj,
              layer.memory_attn.o_proj):
        m.to(bf)
    hg = h.to(dev).requires_grad_(True)
    bg = bank.to(dev).requires_grad_(True)
    out, _ = layer(hg, bg, return_losses=False)
    (out.float() * dO.to(dev)).sum().backward()
    idx_star, _, _ = layer.route(hg.detach(), return_losses=False)
    sel = idx_star[:, S:].cpu().long()                       # global chapter ids of the routed slots

    # routing: distinct, and a top-K of the fp64 logits up to the tie band
    logits64 = O.linear(O.sequence_pool(h.double()), Wr.double(), br.double())
    routed = logits64[:, S:]
    assert all(torch.unique(sel[b]).numel() == K for b in range(B))
    assert int(sel.min()) >= S
    kth = torch.topk(routed, K, dim=-1).values[:, -1:]
    assert bool((routed.gather(1, sel - S) >= kth - 1e-5).all()), "routed chapters are not a top-k of the logits"

    # output and gradients: oracle chain on the GPU's chapter choice (fp32, CPU)
    leaves = [t.float().clone().requires_grad_(True) for t in (h, bank, Wr, br, Wq, Wk, Wv, Wo)]
    hf, bankf, Wrf, brf, Wqf, Wkf, Wvf, Wof = leaves
    logits = O.linear(O.sequence_pool(hf), Wrf, brf)
    probs = torch.softmax(logits, dim=-1)
    p = torch.cat([torch.zeros_like(probs[:, :S]), probs[:, S:]], dim=-1)
    p = p / p.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    w = p.gather(1, sel)
    w = w / w.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    ci, cw = O.prepend_shared_chapters(sel, w, num_chapters=C, num_shared_chapters=S, routed_scaling_factor=SCALE)
    assert torch.equal(ci, idx_star.cpu().long())
    # the oracle's row indices; rows taken by plain indexing (the same rows as its batched
    # gather, whose backward would materialise a (B, 262208, 768) gradient)
    with torch.no_grad():
        _, rows = O.gather_chapters(bankf, ci, T)
    mem = bankf[rows]
    ref = O.cross_attention(hf, O.weight_memory(mem, cw, T), Wqf, Wkf, Wvf, Wof, H, H)
    (ref * dO).sum().backward()

    assert_parity(out, ref.detach(), bf, "out")
    got = [hg.grad, bg.grad, layer.router.router.weight.grad, layer.router.router.bias.grad,
           layer.memory_attn.q_proj.weight.grad, layer.memory_attn.k_proj.weight.grad,
           layer.memory_attn.v_proj.weight.grad, layer.memory_attn.o_proj.weight.grad]
    names = ["dh", "dbank", "dWr", "dbr", "dWq", "dWk", "dWv", "dWo"]
    for n, gr, r in zip(names, got, leaves):
        assert_parity(gr, r.grad, bf, n)


def test_config3_full_size_forward_backward(gpu_device):
    """Rescaled weights (bank x25 of the recipe, projections d^-1/2) so that the attention is
    far from uniform and every gradient is well above bf16 rounding of its inputs."""
    print("full-size config 3 forward + backward (rescaled)", flush=True)
    bf = torch.bfloat16
    g = torch.Generator().manual_seed(3)
    h = torch.randn(B, L, D, generator=g).to(bf)
    bank = (torch.randn(C * T, D, generator=g) * 0.5).to(bf)
    Wr = torch.randn(C, D, generator=g) * 0.02
    br = torch.randn(C, generator=g) * 0.01
    Wq, Wk, Wv, Wo = ((torch.randn(D, D, generator=g) * D ** -0.5).to(bf) for _ in range(4))
    dO = torch.randn(B, L, D, generator=g)
    _config3_check(gpu_device, h, bank, Wr, br, Wq, Wk, Wv, Wo, dO)


def test_config3_recipe_forward_backward(gpu_device):
    """BASELINE's input recipe at config 3: hidden states N(0,1), bank and every weight
    N(0,0.02), router bias 0, o_proj not zeroed, upstream gradient N(0,1) (seed 1)."""
    print("full-size config 3 forward + backward (BASELINE recipe)", flush=True)
    bf = torch.bfloat16
    g = torch.Generator().manual_seed(0)
    h = torch.randn(B, L, D, generator=g).to(bf)
    bank = (torch.randn(C * T, D, generator=g) * 0.02).to(bf)
    Wr = torch.randn(C, D, generator=g) * 0.02
    br = torch.zeros(C)
    Wq, Wk, Wv, Wo = ((torch.randn(D, D, generator=g) * 0.02).to(bf) for _ in range(4))
    dO = torch.randn(B, L, D, generator=torch.Generator().manual_seed(1))
    _config3_check(gpu_device, h, bank, Wr, br, Wq, Wk, Wv, Wo, dO)


def test_config5_full_size_decode(gpu_device):
    print("full-size config 5 decode", flush=True)
    from memory_amd.decode import DecodeRouting, MemoryDecodeCache, memory_decode_step
    from memory_amd.memory_attention import MemoryCrossAttention
    dev = gpu_device
    bf = torch.bfloat16
    Bd = 64
    g = torch.Generator().manual_seed(5)
    h = torch.randn(Bd, 1, D, generator=g).to(bf)
    bank = (torch.randn(C * T, D, generator=g) * 0.5).to(bf)
    Wq, Wk, Wv, Wo = ((torch.randn(D, D, generator=g) * D ** -0.5).to(bf) for _ in range(4))
    logits = torch.randn(Bd, C, generator=g) * 2
    idx, w, _ = O.route_sequence(logits, K, S)
    ci, cw = O.prepend_shared_chapters(idx, w, num_chapters=C, num_shared_chapters=S, routed_scaling_factor=SCALE)

    attn = MemoryCrossAttention(D, H, H, wo_init_zero=False)
    with torch.no_grad():
        for lin, W in ((attn.q_proj, Wq), (attn.k_proj, Wk), (attn.v_proj, Wv), (attn.o_proj, Wo)):
            lin.weight.copy_(W.float())
    attn = attn.to(dev, bf)
    cache = MemoryDecodeCache(bank.to(dev), attn.k_proj.weight, attn.v_proj.weight, num_chapters=C,
                              tokens_per_chapter=T, num_kv_heads=H, dtype=bf)
    routing = DecodeRouting(ci.to(dev), cw.to(dev), C)
    out = memory_decode_step(attn, h.to(dev), cache, routing)
    ref = O.decode_step(h.float(), bank.float(), ci, cw.float(), Wq.float(), Wk.float(), Wv.float(), Wo.float(),
                        H=H, HK=H, T=T, S=S)
    assert_parity(out, ref, torch.bfloat16, "decode output")


def test_config4_widths_token_layer(gpu_device):
    """The token-level layer at config 4's widths (d=768, 12 heads, the 4,097-chapter bank,
    S=1 + k=16, v4 MoE combine) on 256 tokens: every routed chapter's (chapter, head) unit holds
    one or two rows.  Routing: a top-16 of the logits (GEMM operands rounded to bf16 as on the
    GPU) up to a 1e-5 tie band; output and every gradient against the oracle's token layer
    (token_routed_preproj) on the GPU's chapter choice."""
    print("config-4 widths token layer", flush=True)
    from memory_amd.model import TokenRoutedMemoryLayer
    dev = gpu_device
    bf = torch.bfloat16
    Lq, K4 = 256, 16
    g = torch.Generator().manual_seed(4)
    h = torch.randn(1, Lq, D, generator=g).to(bf)
    bank = (torch.randn(C * T, D, generator=g) * 0.5).to(bf)
    Wr = (torch.randn(C, D, generator=g) * 0.02).to(bf).float()   # the router GEMM rounds W to bf16
    br = torch.randn(C, generator=g) * 0.01
    Wq, Wk, Wv, Wo = ((torch.randn(D, D, generator=g) * D ** -0.5).to(bf) for _ in range(4))
    dO = torch.randn(1, Lq, D, generator=g)

    layer = TokenRoutedMemoryLayer(D, H, C, T, K4, num_shared_chapters=S, routed_scaling_factor=SCALE,
                                   weighted=True, kernel_version="v4", wo_init_zero=False)
    with torch.no_grad():
        layer.router.router.weight.copy_(Wr)
        layer.router.router.bias.copy_(br)
        for lin, W in ((layer.memory_attn.q_proj, Wq), (layer.memory_attn.k_proj, Wk),
                       (layer.memory_attn.v_proj, Wv), (layer.memory_attn.o_proj, Wo)):
            lin.weight.copy_(W.float())
    layer = layer.to(dev)
    for m in (layer.memory_attn.q_proj, layer.memory_attn.k_proj, layer.memory_attn.v_proj,
              layer.memory_attn.o_proj):
        m.to(bf)
    hg = h.to(dev).requires_grad_(True)
    bg = bank.to(dev).requires_grad_(True)
    out, _ = layer(hg, bg, return_losses=False)
    (out.float() * dO.to(dev)).sum().backward()
    idx, _, _ = layer.router.route_token_level(hg.detach(), return_losses=False, exclude_prefix_chapters=S)
    idx = idx.cpu().long()                                          # (1, Lq, K4) global ids

    logits64 = O.linear(h.double(), Wr.double(), br.double())[..., S:]
    assert int(idx.min()) >= S
    assert all(torch.unique(idx[0, t]).numel() == K4 for t in range(Lq))
    kth = torch.topk(logits64, K4, dim=-1).values[..., -1:]
    assert bool((logits64.gather(-1, idx - S) >= kth - 1e-5).all()), "routed chapters are not a top-k"

    leaves = [t.float().clone().requires_grad_(True) for t in (h, bank, Wr, br, Wq, Wk, Wv, Wo)]
    hf, bankf, Wrf, brf, Wqf, Wkf, Wvf, Wof = leaves
    probs = torch.softmax(O.linear(hf, Wrf, brf), dim=-1)
    routed = probs[..., S:] / probs[..., S:].sum(dim=-1, keepdim=True).clamp_min(1e-12)
    w = routed.gather(-1, idx - S)
    w = w / w.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    pre = O.token_routed_preproj(hf, bankf[: S * T], bankf[S * T:], idx - S, w, T, SCALE, Wqf, Wkf, Wvf, H, H)
    ref = O.linear(pre, Wof)
    (ref * dO).sum().backward()

    assert_parity(out, ref.detach(), torch.bfloat16, "out")
    got = [hg.grad, bg.grad, layer.router.router.weight.grad, layer.router.router.bias.grad,
           layer.memory_attn.q_proj.weight.grad, layer.memory_attn.k_proj.weight.grad,
           layer.memory_attn.v_proj.weight.grad, layer.memory_attn.o_proj.weight.grad]
    names = ["dh", "dbank", "dWr", "dbr", "dWq", "dWk", "dWv", "dWo"]
    for n, gr, r in zip(names, got, leaves):
        assert_parity(gr, r.grad, torch.bfloat16, n)


def test_config4_full_size_sampled(gpu_device):
    """The token-level layer at config 4's full size (B=4, L=2048: 8,192 tokens, every
    (chapter, head) unit holding ~32 rows) forward and backward on the GPU.  The upstream
    gradient is zero except on 256 sampled tokens, so the output rows of those tokens and every
    gradient (a sum over the sampled tokens only) can be checked against the oracle's token
    layer (token_routed_preproj, memory_attention.py:480-716) run on those tokens alone; the
    routing of the sampled tokens is checked as a top-16 of their logits; h's gradient is
    exactly zero on every other token."""
    print("full-size config 4 forward + backward, sampled rows", flush=True)
    from memory_amd.model import TokenRoutedMemoryLayer
    dev = gpu_device
    bf = torch.bfloat16
    B4, L4, K4, NS = 4, 2048, 16, 256
    g = torch.Generator().manual_seed(44)
    h = torch.randn(B4, L4, D, generator=g).to(bf)
    bank = (torch.randn(C * T, D, generator=g) * 0.5).to(bf)
    Wr = (torch.randn(C, D, generator=g) * 0.02).to(bf).float()   # the router GEMM rounds W to bf16
    br = torch.randn(C, generator=g) * 0.01
    Wq, Wk, Wv, Wo = ((torch.randn(D, D, generator=g) * D ** -0.5).to(bf) for _ in range(4))
    flat = torch.randperm(B4 * L4, generator=g)[:NS].sort().values
    dO = torch.zeros(B4 * L4, D)
    dO[flat] = torch.randn(NS, D, generator=g)
    dO = dO.view(B4, L4, D)

    layer = TokenRoutedMemoryLayer(D, H, C, T, K4, num_shared_chapters=S, routed_scaling_factor=SCALE,
                                   weighted=True, kernel_version="v4", wo_init_zero=False)
    with torch.no_grad():
        layer.router.router.weight.copy_(Wr)
        layer.router.router.bias.copy_(br)
        for lin, W in ((layer.memory_attn.q_proj, Wq), (layer.memory_attn.k_proj, Wk),
                       (layer.memory_attn.v_proj, Wv), (layer.memory_attn.o_proj, Wo)):
            lin.weight.copy_(W.float())
    layer = layer.to(dev)
    for m in (layer.memory_attn.q_proj, layer.memory_attn.k_proj, layer.memory_attn.v_proj,
              layer.memory_attn.o_proj):
        m.to(bf)
    hg = h.to(dev).requires_grad_(True)
    bg = bank.to(dev).requires_grad_(True)
    out, _ = layer(hg, bg, return_losses=False)
    (out.float() * dO.to(dev)).sum().backward()
    assert bool(torch.isfinite(out).all())
    idx, _, _ = layer.router.route_token_level(hg.detach(), return_losses=False, exclude_prefix_chapters=S)
    idx = idx.reshape(B4 * L4, K4)[flat.to(dev)].cpu().long()        # (NS, K4) global ids

    hs = h.reshape(B4 * L4, D)[flat].unsqueeze(0)                     # (1, NS, D) sampled tokens
    logits64 = O.linear(hs.double(), Wr.double(), br.double())[0, :, S:]
    assert int(idx.min()) >= S
    assert all(torch.unique(idx[t]).numel() == K4 for t in range(NS))
    kth = torch.topk(logits64, K4, dim=-1).values[:, -1:]
    assert bool((logits64.gather(-1, idx - S) >= kth - 1e-5).all()), "routed chapters are not a top-k"

    # the oracle on the sampled tokens, over the chapters they selected (compacted: the same
    # per-(token, chapter) softmaxes, K / V projected only for those chapters)
    uc, inv = torch.unique(idx - S, return_inverse=True)
    leaves = [t.float().clone().requires_grad_(True) for t in (hs, bank, Wr, br, Wq, Wk, Wv, Wo)]
    hf, bankf, Wrf, brf, Wqf, Wkf, Wvf, Wof = leaves
    probs = torch.softmax(O.linear(hf, Wrf, brf), dim=-1)
    routed = probs[..., S:] / probs[..., S:].sum(dim=-1, keepdim=True).clamp_min(1e-12)
    w = routed.gather(-1, (idx - S).unsqueeze(0))
    w = w / w.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    rows = (S + uc).unsqueeze(-1) * T + torch.arange(T)
    routed_rows = bankf[rows.reshape(-1)]
    pre = O.token_routed_preproj(hf, bankf[: S * T], routed_rows, inv.view(1, NS, K4), w, T, SCALE,
                                 Wqf, Wkf, Wvf, H, H)
    ref = O.linear(pre, Wof)
    (ref * dO.reshape(B4 * L4, D)[flat].unsqueeze(0)).sum().backward()

    assert_parity(out.reshape(B4 * L4, D)[flat.to(dev)], ref[0].detach(), bf, "out (sampled rows)")
    dh = hg.grad.reshape(B4 * L4, D)
    assert_parity(dh[flat.to(dev)], hf.grad[0], bf, "dh (sampled rows)")
    rest = torch.ones(B4 * L4, dtype=torch.bool)
    rest[flat] = False
    assert int(torch.count_nonzero(dh[rest.to(dev)])) == 0, "dh must be zero where the upstream gradient is"
    got = [bg.grad, layer.router.router.weight.grad, layer.router.router.bias.grad,
           layer.memory_attn.q_proj.weight.grad, layer.memory_attn.k_proj.weight.grad,
           layer.memory_attn.v_proj.weight.grad, layer.memory_attn.o_proj.weight.grad]
    names = ["dbank", "dWr", "dbr", "dWq", "dWk", "dWv", "dWo"]
    for n, gr, r in zip(names, got, leaves[1:]):
        assert_parity(gr, r.grad, bf, n)
