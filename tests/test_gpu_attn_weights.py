"""GPU parity of MemoryCrossAttention.forward(return_attn_weights=True) (the weights of
memory_attention.py:437-447, moc_xattn_weights) against the oracle: a dense memory (per batch and
shared), and the sequence-routed state (gathered, omega-weighted chapters, GQA, a row count that
is not a multiple of 64), in fp32 and bf16; the output equals the call without weights."""

import pytest
import torch

import oracle as O
from helpers import assert_parity, gen

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", ["dense3d", "dense2d", "routed"])
def test_attention_weights_match_oracle(gpu_device, dtype, case):
    print(f"attention weights case={case} dtype={dtype}", flush=True)
    from memory_amd.memory_attention import MemoryCrossAttention
    dev = gpu_device
    g = gen(61 + len(case))
    B, L, H, HK, T = 3, 100, 4, 2, 64
    d = H * 64
    attn = MemoryCrossAttention(d, H, HK, wo_init_zero=False)
    with torch.no_grad():
        for lin in (attn.q_proj, attn.k_proj, attn.v_proj, attn.o_proj):
            lin.weight.copy_(torch.randn(lin.weight.shape, generator=g) / d ** 0.5)
    Wq, Wk = attn.q_proj.weight.detach().clone(), attn.k_proj.weight.detach().clone()
    attn = attn.to(dev, dtype)
    h = torch.randn(B, L, d, generator=g)
    rd = lambda t: t.to(dtype).double()
    if case == "routed":
        C, NS = 9, 4
        bank = torch.randn(C * T, d, generator=g)
        idx = torch.stack([torch.randperm(C, generator=g)[:NS] for _ in range(B)])
        omega = torch.rand(B, NS, generator=g) + 0.1
        state = {"bank": bank.to(dev, dtype), "chapter_indices": idx.to(dev), "chapter_weights": omega.to(dev),
                 "num_chapters": C, "tokens_per_chapter": T}
        kw = dict(routed_memory_state=state)
        mem, _ = O.gather_chapters(rd(bank), idx, T)
        mem = O.weight_memory(mem, omega.double(), T)
    else:
        N = 192
        mem = torch.randn(B, N, d, generator=g) if case == "dense3d" else torch.randn(N, d, generator=g)
        kw = dict(memory=mem.to(dev, dtype))
        mem = rd(mem)
    out_w, P = attn(h.to(dev, dtype), return_attn_weights=True, **kw)
    out, none = attn(h.to(dev, dtype), **kw)
    assert none is None and torch.equal(out_w, out)
    ref = O.attention_weights(rd(h), mem, rd(Wq), rd(Wk), H, HK)
    assert P.dtype == dtype and P.shape == ref.shape
    assert_parity(P, ref, dtype, f"{case} attention weights")


def test_attention_weights_token_path_rejected(gpu_device):
    from memory_amd.memory_attention import MemoryCrossAttention
    attn = MemoryCrossAttention(128, 2).to(gpu_device)
    h = torch.randn(1, 4, 128, device=gpu_device)
    with pytest.raises(ValueError, match="token_routing_state"):
        attn(h, token_routing_state={"token_chapter_indices": torch.zeros(1, 4, 1, dtype=torch.long)},
             return_attn_weights=True)
