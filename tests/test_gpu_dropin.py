"""The paths an unmodified MemoryTransformer takes into the layer, on the GPU against the oracle.

* MemoryCrossAttention.forward(h, memory=(B, (S+k)*T, d)): the omega-weighted gathered memory
  that MemoryTransformer.forward builds (model.py:677-692) and MemoryTransformerBlock passes on
  (memory_block.py:552-557), forward and backward (h, memory -- which carries the bank's and the
  router's gradients upstream -- and the four projections), at config 1 and at config 3's
  widths (d=768, 12 heads, 65 chapters).
* The token-routing kernel loader (token_routing_kernel.py:35-142): the functions it returns
  for v1..v5 run the sparse kernels; checked against the reference's naive references.
* MemoryTransformer._select_routed_chapters_from_probs (model.py:331-354), ties included.
* MemoryCrossAttentionWithRouting (memory_attention.py:901-1054), weighted and unweighted,
  with a 2-D bank or an already routed (B, k*T, d) memory.

Gate: fp32 every element within 1e-4 relative, bf16 max-abs 2e-2 (tests/helpers.py)."""

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_parity, gen

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(gpu_device):
    from memory_amd import _lib
    _lib.lib()
    return gpu_device


def _attn(dev, dtype, d, H, Wq, Wk, Wv, Wo):
    from memory_amd.memory_attention import MemoryCrossAttention
    m = MemoryCrossAttention(d, H, H, wo_init_zero=False)
    with torch.no_grad():
        for lin, W in ((m.q_proj, Wq), (m.k_proj, Wk), (m.v_proj, Wv), (m.o_proj, Wo)):
            lin.weight.copy_(W)
    return m.to(dev, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,Lq,d,H,C,k", [(2, 128, 256, 4, 33, 4), (2, 256, 768, 12, 4097, 64)])
def test_memory_argument_weighted_gathered(dev, dtype, B, Lq, d, H, C, k):
    """forward(h, memory=omega-weighted gathered chapters), the call model.py:689-692 ->
    memory_block.py:552-557 makes, against the oracle's cross-attention over the same memory."""
    print(f"memory= path dtype={dtype} B={B} L={Lq} d={d} H={H} C={C} k={k}", flush=True)
    T, S, s = 64, 1, 2.5
    g = gen(100 + d)
    h = torch.randn(B, Lq, d, generator=g)
    bank = torch.randn(C * T, d, generator=g) * 0.5
    Wq, Wk, Wv, Wo = (torch.randn(d, d, generator=g) * d ** -0.5 for _ in range(4))
    logits = torch.randn(B, C, generator=g)
    idx, w, _ = O.route_sequence(logits, k, S)
    ci, cw = O.prepend_shared_chapters(idx, w, num_chapters=C, num_shared_chapters=S, routed_scaling_factor=s)
    mem = O.weight_memory(O.gather_chapters(bank, ci, T)[0], cw, T)        # (B, (S+k)*T, d)
    dO = torch.randn(B, Lq, d, generator=g)
    if dtype != torch.float32:
        h, mem, Wq, Wk, Wv, Wo = (t.to(dtype).float() for t in (h, mem, Wq, Wk, Wv, Wo))

    m = _attn(dev, dtype, d, H, Wq, Wk, Wv, Wo)
    hg = h.to(dev, dtype).requires_grad_(True)
    mg = mem.to(dev, dtype).requires_grad_(True)
    out, attn_w = m(hg, memory=mg)
    assert attn_w is None and out.shape == (B, Lq, d)
    (out.float() * dO.to(dev)).sum().backward()

    ref_dt = torch.float64 if dtype == torch.float32 else torch.float32
    leaves = [t.to(ref_dt).clone().requires_grad_(True) for t in (h, mem, Wq, Wk, Wv, Wo)]
    ref = O.cross_attention(leaves[0], leaves[1], *leaves[2:], H, H)
    (ref * dO.to(ref_dt)).sum().backward()
    assert_parity(out, ref.detach(), dtype, "out")
    got = [hg.grad, mg.grad, m.q_proj.weight.grad, m.k_proj.weight.grad, m.v_proj.weight.grad,
           m.o_proj.weight.grad]
    for n, gr, r in zip(["dh", "dmemory", "dWq", "dWk", "dWv", "dWo"], got, leaves):
        assert_parity(gr, r.grad, dtype, n)


# ---------------------------------------------------------------- the kernel loader

def _fsa_inputs(B=1, Tq=96, HQ=4, HK=2, M=9, S=3, seed=0):
    g = gen(seed)
    q = torch.randn(B, Tq, HQ, 64, generator=g)
    k = torch.randn(B, M * 64, HK, 64, generator=g)
    v = torch.randn(B, M * 64, HK, 64, generator=g)
    idx = torch.stack([torch.randperm(M, generator=g)[:S] for _ in range(B * Tq * HK)]).view(B, Tq, HK, S)
    w = torch.rand(B, Tq, S, generator=g) + 0.1
    w = w / w.sum(-1, keepdim=True)
    return q, k, v, idx, w


@pytest.mark.parametrize("version", ["v1", "v2", "v3", "4", "kernel_v5"])
def test_loader_functions_run_the_kernels(dev, version):
    """Every version's functions from the loader against the reference's naive references
    (kernels-final/benchmark_kernels_final.py:206-337): unweighted joint softmax for
    get_token_routing_kernel_fn; the per-chapter MoE (v4) or the joint log-bias (v5) for
    get_token_routing_weighted_kernel_fn, which is None for v1-v3."""
    from memory_amd import token_routing_kernel as trk
    print(f"loader version={version}", flush=True)
    q, k, v, idx, w = _fsa_inputs(seed=sum(map(ord, version)))
    fn = trk.get_token_routing_kernel_fn(version)
    out = fn(q.to(dev), k.to(dev), v.to(dev), idx.to(dev).int(), 64, disable_causal_mask=True)
    ref = O.naive_reference_unweighted(q.double(), k.double(), v.double(), idx, 64, 64 ** -0.5)
    assert_parity(out, ref, torch.float32, f"{version} unweighted")
    wfn = trk.get_token_routing_weighted_kernel_fn(version)
    ver = trk.normalize_kernel_version(version)
    if ver in ("v1", "v2", "v3"):
        assert wfn is None
        return
    out = wfn(q.to(dev), k.to(dev), v.to(dev), idx.to(dev).int(), w.to(dev), 64, disable_causal_mask=True)
    naive = O.naive_reference_weighted if ver == "v4" else O.naive_reference_weighted_joint_bias
    ref = naive(q.double(), k.double(), v.double(), idx, w.double(), 64, 64 ** -0.5)
    assert_parity(out, ref, torch.float32, f"{version} weighted")


# ------------------------------------------------------- _select_routed_chapters_from_probs

@pytest.mark.parametrize("B,C,S,k", [(4, 33, 1, 4), (8, 4097, 1, 64), (3, 50, 0, 7), (2, 300, 2, 298),
                                     (5, 33, 1, 40), (3, 9, 9, 2)])
def test_select_routed_chapters_from_probs(dev, B, C, S, k):
    """memory_amd.model.select_routed_chapters_from_probs against the oracle restatement of
    model.py:331-354 (mask the shared prefix, renormalise, top-k, renormalise)."""
    from memory_amd.model import select_routed_chapters_from_probs
    print(f"select_from_probs B={B} C={C} S={S} k={k}", flush=True)
    probs = torch.softmax(torch.randn(B, C, generator=gen(C + k)) * 3, dim=-1)
    idx, w = select_routed_chapters_from_probs(probs.to(dev), k, S)
    ri, rw = O.select_routed_chapters_from_probs(probs, k, S)       # fp32, as the reference runs it
    assert idx.dtype == torch.long and idx.shape == ri.shape
    assert torch.equal(idx.cpu(), ri)
    if ri.numel():
        assert_parity(w, rw.double(), torch.float32, "weights")
    # gradients reach the probabilities through the renormalised weights, as in the reference
    pg = probs.to(dev).requires_grad_(True)
    pr = probs.double().requires_grad_(True)
    dw = torch.randn(B, ri.shape[1], generator=gen(7), dtype=torch.float64)
    if ri.numel():
        (select_routed_chapters_from_probs(pg, k, S)[1] * dw.float().to(dev)).sum().backward()
        (O.select_routed_chapters_from_probs(pr, k, S)[1] * dw).sum().backward()
        assert_parity(pg.grad, pr.grad, torch.float32, "dprobs")


def test_select_routed_chapters_from_probs_ties(dev):
    """Equal probabilities: the lower chapter id comes first (the documented tie rule)."""
    from memory_amd.model import select_routed_chapters_from_probs
    levels = torch.randint(0, 4, (6, 129), generator=gen(9)).double()
    probs = torch.softmax(levels, dim=-1)                 # ~32 copies of each value per row
    idx, w = select_routed_chapters_from_probs(probs.float().to(dev), 40, 1)
    masked = np.where(np.arange(129)[None, :] < 1, -np.inf, probs.float().numpy())
    assert np.array_equal(idx.cpu().numpy(), O.topk_desc_numpy(masked, 40))
    ri, rw = O.select_routed_chapters_from_probs(probs.float(), 40, 1)
    assert torch.equal(idx.cpu(), ri)
    assert_parity(w, rw.double(), torch.float32, "tie weights")


# ---------------------------------------------------------- MemoryCrossAttentionWithRouting

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("weighted", [True, False])
@pytest.mark.parametrize("routed_memory", [False, True])
@pytest.mark.parametrize("T", [64, 128])
def test_memory_cross_attention_with_routing(dev, dtype, weighted, routed_memory, T):
    """T = 128: a chapter is two 64-row blocks (the weighted form one joint softmax per slot)."""
    from memory_amd.memory_attention import MemoryCrossAttentionWithRouting
    print(f"with-routing dtype={dtype} weighted={weighted} routed_memory={routed_memory} T={T}", flush=True)
    B, Lq, d, H, C, k = 2, 100, 256, 4, 17 if T == 64 else 9, 3
    g = gen(31)
    h = torch.randn(B, Lq, d, generator=g)
    bank = torch.randn(C * T, d, generator=g) * 0.5
    Wq, Wk, Wv, Wo = (torch.randn(d, d, generator=g) * d ** -0.5 for _ in range(4))
    ci = torch.stack([torch.randperm(C, generator=g)[:k] for _ in range(B)])
    cw = torch.rand(B, k, generator=g) + 0.05
    cw = cw / cw.sum(-1, keepdim=True)
    dO = torch.randn(B, Lq, d, generator=g)
    if dtype != torch.float32:
        h, bank, Wq, Wk, Wv, Wo = (t.to(dtype).float() for t in (h, bank, Wq, Wk, Wv, Wo))
    mem = O.gather_chapters(bank, ci, T)[0] if routed_memory else bank

    m = MemoryCrossAttentionWithRouting(d, H, C, T, k, wo_init_zero=False)
    with torch.no_grad():
        for lin, W in ((m.attention.q_proj, Wq), (m.attention.k_proj, Wk), (m.attention.v_proj, Wv),
                       (m.attention.o_proj, Wo)):
            lin.weight.copy_(W)
    m = m.to(dev, dtype)
    hg = h.to(dev, dtype).requires_grad_(True)
    mg = mem.to(dev, dtype).requires_grad_(True)
    out, aw = m(hg, mg, ci.to(dev), cw.to(dev) if weighted else None)
    assert aw is None
    (out.float() * dO.to(dev)).sum().backward()

    ref_dt = torch.float64 if dtype == torch.float32 else torch.float32
    leaves = [t.to(ref_dt).clone().requires_grad_(True) for t in (h, mem, Wq, Wk, Wv, Wo)]
    ref = O.moe_with_routing(leaves[0], leaves[1], ci, cw.to(ref_dt) if weighted else None, T, *leaves[2:], H, H)
    (ref * dO.to(ref_dt)).sum().backward()
    assert_parity(out, ref.detach(), dtype, "out")
    got = [hg.grad, mg.grad, m.attention.q_proj.weight.grad, m.attention.k_proj.weight.grad,
           m.attention.v_proj.weight.grad, m.attention.o_proj.weight.grad]
    for n, gr, r in zip(["dh", "dmemory", "dWq", "dWk", "dWv", "dWo"], got, leaves):
        assert_parity(gr, r.grad, dtype, n)
