"""A MemoryStack loaded from a reference-format checkpoint runs its memory sublayer like the
oracle with the same weights (routing on the block input, memory_layernorm + memory
cross-attention + residual on the hidden states: model.py:609-692, memory_block.py:549-558),
and the decode K/V cache survives a save / load round trip bit for bit."""

import pytest
import torch

import oracle as O
from helpers import assert_parity, assert_rel, gen
from test_checkpoint import _config, _reference_state_dict

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(gpu_device):
    from memory_amd import _lib
    _lib.lib()
    return gpu_device


@pytest.mark.parametrize("use_rms", [True, False])
def test_loaded_stack_layer_matches_oracle(dev, use_rms):
    print(f"loaded memory stack layer rms={use_rms}", flush=True)
    from memory_amd.checkpoint import MemoryStack
    cfg = _config(use_rms)
    sd = _reference_state_dict(cfg, seed=3)
    for k in list(sd):
        if ".memory_attn." in k:
            sd[k] = sd[k] * 0.125                      # keep attention logits moderate
        if k.startswith("routers."):
            sd[k] = sd[k] * 0.1
    stack = MemoryStack.from_config(cfg)
    stack.load_reference_state_dict(sd)
    stack = stack.to(dev)
    layer, bank_idx = 2, stack.bank_of[2]
    g0 = gen(9)
    B, L, d = 2, 90, cfg["model"]["hidden_dim"]
    block_in = torch.randn(B, L, d, generator=g0)
    hidden = torch.randn(B, L, d, generator=g0)
    out, _ = stack(layer, block_in.to(dev), hidden.to(dev), return_losses=False)
    with torch.no_grad():
        idx_gpu, _, _ = stack.routers[str(layer)](block_in.to(dev), return_losses=False, exclude_prefix_chapters=1)
    m = cfg["memory"]
    C, k, S, T = m["num_chapters"], m["top_k_chapters"], m["num_shared_chapters"], 64
    Wr, br = sd[f"routers.{layer}.router.weight"].double(), sd[f"routers.{layer}.router.bias"].double()
    logits = O.linear(O.sequence_pool(block_in.double()), Wr, br)
    idx, w, _ = O.route_sequence(logits, k, S)
    assert torch.equal(idx_gpu.cpu().long(), idx.long())
    ci, cw = O.prepend_shared_chapters(idx, w, num_chapters=C, num_shared_chapters=S, routed_scaling_factor=2.5)
    bank = sd[f"memory_banks.{bank_idx}.base_bank.memory"].double()
    mem, _ = O.gather_chapters(bank, ci, T)
    mem = O.weight_memory(mem, cw, T)
    pre = f"layers.{layer}."
    ref = O.memory_sublayer(hidden.double(), sd[pre + "memory_layernorm.weight"].double(),
                            None if use_rms else sd[pre + "memory_layernorm.bias"].double(), 1e-5, use_rms, mem,
                            *(sd[pre + f"memory_attn.{p}_proj.weight"].double() for p in "qkvo"), 2, 2)
    assert_parity(out, ref, torch.float32, "memory sublayer output")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_cache_save_load(dev, dtype, tmp_path):
    print(f"decode cache file round trip {dtype}", flush=True)
    from memory_amd.decode import DecodeRouting, MemoryDecodeCache, decode_attention
    C, T, d, HK = 11, 64, 128, 2
    g0 = gen(13)
    bank = torch.randn(C * T, d, generator=g0).to(dev, dtype)
    wk = (torch.randn(HK * 64, d, generator=g0) * 0.1).to(dev, dtype)
    wv = (torch.randn(HK * 64, d, generator=g0) * 0.1).to(dev, dtype)
    cache = MemoryDecodeCache(bank, wk, wv, num_chapters=C, tokens_per_chapter=T, num_kv_heads=HK, dtype=dtype)
    path = str(tmp_path / "layer2.kv.safetensors")
    cache.save(path)
    back = MemoryDecodeCache.load(path, dev)
    assert back.dtype == dtype and (back.num_chapters, back.T, back.HK) == (C, T, HK)
    assert torch.equal(back.k_tiles, cache.k_tiles) and torch.equal(back.v_tiles, cache.v_tiles)
    idx = torch.tensor([[0, 3, 7], [0, 10, 3]], device=dev, dtype=torch.int32)
    om = torch.tensor([[0.5, 0.3, 0.2], [0.4, 0.4, 0.2]], device=dev)
    routing = DecodeRouting(idx, om, C)
    q = torch.randn(2, HK, 64, generator=g0).to(dev, dtype)
    assert torch.equal(decode_attention(q, back, routing), decode_attention(q, cache, routing))


def test_load_and_export_with_bank_optimizer(dev):
    """A stack whose bank is stepped by BankAdamW (bf16 mirror read by the kernels): exporting
    brings every chapter to the last step first, and loading reference weights refreshes the
    mirror, so the next forward reads the loaded bank (the fine-tune flow of
    training/trainer.py:668-709, weights loaded into a model whose optimizer exists)."""
    print("load / export with BankAdamW", flush=True)
    from memory_amd.bank_optim import BankAdamW
    from memory_amd.checkpoint import MemoryStack
    cfg = _config(True)
    sd = _reference_state_dict(cfg, seed=3)
    for k in list(sd):
        if ".memory_attn." in k:
            sd[k] = sd[k] * 0.125
        if k.startswith("routers."):
            sd[k] = sd[k] * 0.1
    stack = MemoryStack.from_config(cfg).to(dev)
    layer = 2
    bank = stack.bank_for(layer)
    key = f"memory_banks.{stack.bank_of[layer]}.base_bank.memory"
    opt = BankAdamW(bank, 64, lr=1e-2, weight_decay=0.1, mirror_dtype=torch.bfloat16)
    g0 = gen(21)
    B, L, d = 2, 90, cfg["model"]["hidden_dim"]
    for _ in range(3):                       # chapters go stale, the mirror moves away from sd
        x = torch.randn(B, L, d, generator=g0).to(dev)
        out, _ = stack(layer, x, x, return_losses=False)
        out.float().pow(2).sum().backward()
        opt.step()
        opt.zero_grad()
    stale = bank.detach().clone()
    exported = stack.reference_state_dict()[key].clone()
    assert not torch.equal(exported, stale), "export must bring stale chapters to the last step"
    opt.flush()
    assert torch.equal(exported, bank.detach())

    stack.load_reference_state_dict(sd)
    assert torch.equal(bank.detach().cpu(), sd[key].float())
    assert torch.equal(opt.mirror.cpu(), sd[key].to(torch.bfloat16))
    block_in = torch.randn(B, L, d, generator=g0)
    hidden = torch.randn(B, L, d, generator=g0)
    stack.eval()
    m = cfg["memory"]
    C, k, S, T = m["num_chapters"], m["top_k_chapters"], m["num_shared_chapters"], 64
    Wr, br = sd[f"routers.{layer}.router.weight"].double(), sd[f"routers.{layer}.router.bias"].double()
    pre = f"layers.{layer}."
    nw = sd[pre + "memory_layernorm.weight"].double()
    Wqkvo = [sd[pre + f"memory_attn.{p}_proj.weight"].double() for p in "qkvo"]
    for dtype in (torch.float32, torch.bfloat16):
        # fp32 layers read the fp32 bank; bf16 layers read the bf16 mirror refreshed by the load
        rd = (lambda t: t) if dtype == torch.float32 else (lambda t: t.to(dtype).double())
        stack.layers[str(layer)].to(dtype)
        with torch.no_grad():
            out, losses = stack(layer, block_in.to(dev, dtype), hidden.to(dev, dtype))
        assert not losses, "an eval forward returns no router losses (return_losses=self.training)"
        idx, w, _ = O.route_sequence(O.linear(O.sequence_pool(rd(block_in.double())), Wr, br), k, S)
        ci, cw = O.prepend_shared_chapters(idx, w, num_chapters=C, num_shared_chapters=S, routed_scaling_factor=2.5)
        bank_read = rd(sd[key].double())
        mem = O.weight_memory(O.gather_chapters(bank_read, ci, T)[0], cw, T)
        ref = O.memory_sublayer(rd(hidden.double()), nw, None, 1e-5, True, mem, *(rd(W) for W in Wqkvo), 2, 2)
        assert_parity(out.float(), ref, dtype, f"{dtype} output after load")
