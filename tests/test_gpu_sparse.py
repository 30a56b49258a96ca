"""GPU parity of the token-routed sparse attention (the FSA entry points of the
reference's kernels v1-v5 and MemoryCrossAttention's token path) against the
oracle's vectorised restatements of benchmark_kernels_final.py's naive
references, forward and backward (float64 autograd).

fp32: 1e-4 relative max error; bf16: 2e-2 (3e-2 for weight gradients, the
reference harness's bf16 backward tolerance, benchmark_kernels_final.py:676-682)."""

import pytest
import torch

import oracle as O
from helpers import assert_parity, assert_rel, gen

pytestmark = pytest.mark.gpu

REF = {1: O.sparse_attention_unweighted, 2: O.sparse_attention_block_weighted, 0: O.sparse_attention_weighted,
       3: O.sparse_attention_joint_bias}


def _inputs(seed, B, Tq, HQ, HK, M, S, per_head, mode):
    g = gen(seed)
    D = 64
    q = torch.randn(B, Tq, HQ, D, generator=g)
    k = torch.randn(B, M * 64, HK, D, generator=g)
    v = torch.randn(B, M * 64, HK, D, generator=g)
    if per_head:
        idx = torch.stack([torch.stack([torch.randperm(M, generator=g)[:S] for _ in range(HK)])
                           for _ in range(B * Tq)]).view(B, Tq, HK, S)
    else:
        idx = torch.stack([torch.randperm(M, generator=g)[:S] for _ in range(B * Tq)]).view(B, Tq, 1, S)
        idx = idx.expand(B, Tq, HK, S).contiguous()
    if mode == 2:
        w = torch.rand(B, Tq, HK, S, generator=g) + 0.05
    elif mode in (0, 3):
        w = torch.rand(B, Tq, S, generator=g) + 0.05
        w = w / w.sum(-1, keepdim=True)
    else:
        w = None
    dO = torch.randn(B, Tq, HQ, D, generator=g)
    return q, k, v, idx, w, dO


def _ref(mode, q, k, v, idx, w, scale):
    f = REF[mode]
    if mode == 1:
        return f(q, k, v, idx, 64, scale)
    return f(q, k, v, idx, w, 64, scale)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", [0, 1, 2, 3])
# the third case gives every (chapter, kv head) ~130 rows: several 32-row blocks and a ragged last one;
# the last two take the streaming slot combine (more than 68 slots per token; more than 16,384 rows),
# the others the single-round one
@pytest.mark.parametrize("B,Tq,HQ,HK,M,S,per_head", [(2, 40, 2, 2, 6, 3, False), (1, 70, 4, 2, 5, 2, True),
                                                     (1, 200, 2, 2, 3, 2, False), (1, 30, 2, 2, 80, 70, False),
                                                     (1, 2100, 8, 2, 4, 2, False)])
def test_fsa_modes_forward_backward(gpu_device, dtype, mode, B, Tq, HQ, HK, M, S, per_head):
    print(f"fsa mode={mode} dtype={dtype} B={B} Tq={Tq} HQ={HQ} HK={HK} M={M} S={S} per_head={per_head}", flush=True)
    from memory_amd import sparse_attention as SA
    dev = gpu_device
    q, k, v, idx, w, dO = _inputs(31 + mode + 7 * per_head, B, Tq, HQ, HK, M, S, per_head, mode)
    scale = 0.125
    rq, rk, rv = (t.to(dtype).double().requires_grad_(True) for t in (q, k, v))
    rw = None if w is None else w.double().requires_grad_(True)
    ref = _ref(mode, rq, rk, rv, idx, rw, scale)
    (ref * dO.to(dtype).double()).sum().backward()

    gq, gk, gv = (t.to(dev, dtype).requires_grad_(True) for t in (q, k, v))
    gw = None if w is None else w.to(dev).requires_grad_(True)
    idx_d = idx.to(dev, torch.int32)
    kw = dict(softmax_scale=scale, disable_causal_mask=True)
    if mode == 0:
        out = SA.FSA_topk_sparse_attention_weighted_bthd(gq, gk, gv, idx_d, gw, 64, **kw)
    elif mode == 3:
        out = SA.FSA_topk_sparse_attention_weighted_joint_bias_bthd(gq, gk, gv, idx_d, gw, 64, **kw)
    else:
        out = SA.FSA_topk_sparse_attention_bthd(gq, gk, gv, idx_d, 64, block_weights_bths=gw, **kw)
    (out.float() * dO.to(dev)).sum().backward()
    assert_parity(out, ref, dtype, "out")
    assert_parity(gq.grad, rq.grad, dtype, "dq")
    assert_parity(gk.grad, rk.grad, dtype, "dk")
    assert_parity(gv.grad, rv.grad, dtype, "dv")
    if w is not None:
        assert_parity(gw.grad, rw.grad, dtype, "dw")


def test_fsa_out_of_range_chapters_are_skipped(gpu_device):
    """The reference's kernels skip chapter ids outside [0, M) (kernels-final/kernel_v4.py:353):
    for the MoE combine that equals giving the slot weight 0."""
    from memory_amd import sparse_attention as SA
    dev = gpu_device
    q, k, v, idx, w, dO = _inputs(77, 1, 20, 2, 2, 4, 3, False, 0)
    bad = idx.clone()
    bad[0, ::3, :, 1] = 9          # out of range
    bad[0, 1::5, :, 2] = -1
    ref_idx = torch.where((bad < 0) | (bad >= 4), torch.zeros_like(bad), bad)
    ref_w = w.clone()
    ref_w[(bad[:, :, 0, :] < 0) | (bad[:, :, 0, :] >= 4)] = 0.0
    ref = O.sparse_attention_weighted(q.double(), k.double(), v.double(), ref_idx, ref_w.double(), 64, 0.125)
    out = SA.FSA_topk_sparse_attention_weighted_bthd(q.to(dev), k.to(dev), v.to(dev), bad.to(dev, torch.int32),
                                                     w.to(dev), 64, softmax_scale=0.125, disable_causal_mask=True)
    assert_parity(out, ref, torch.float32, "out with skipped slots")


def test_fsa_rejects_unsupported(gpu_device):
    from memory_amd import sparse_attention as SA
    dev = gpu_device
    q = torch.randn(1, 4, 2, 64, device=dev)
    k = torch.randn(1, 128, 2, 64, device=dev)
    idx = torch.zeros(1, 4, 2, 1, dtype=torch.int32, device=dev)
    with pytest.raises(NotImplementedError, match="causal"):
        SA.FSA_topk_sparse_attention_bthd(q, k, k, idx, 64)
    with pytest.raises(ValueError, match="block_size"):
        SA.FSA_topk_sparse_attention_bthd(q, k, k, idx, 32, disable_causal_mask=True)
    with pytest.raises(ValueError, match="block_size"):
        SA.FSA_topk_sparse_attention_weighted_bthd(q, k, k, idx, torch.ones(1, 4, 1, device=dev), 96,
                                                   disable_causal_mask=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode,BS", [(1, 128), (2, 128), (3, 256), (0, 128), (1, 64), (0, 64), (3, 64)])
def test_fsa_block_sizes_and_fp16(gpu_device, dtype, mode, BS):
    """The FSA entry points at block_size 64 m (a block as m consecutive 64-key blocks with the
    block's weight, the MoE combine one joint call per slot; a last block reaching past the
    keys) and with fp16 inputs
    (the fp32 kernels, output rounded to fp16), against the naive references at that block size
    (benchmark_kernels_final.py:206-337 restated in the oracle), gradients included."""
    print(f"fsa block sizes mode={mode} BS={BS} dtype={dtype}", flush=True)
    from memory_amd import sparse_attention as SA
    dev = gpu_device
    g = gen(91 + mode + BS)
    B, Tq, HQ, HK, S = 1, 48, 4, 2, 3
    M = 5
    Tk = M * BS - (64 if BS > 64 else 0)      # the last block is partial when BS > 64
    q = torch.randn(B, Tq, HQ, 64, generator=g)
    k = torch.randn(B, Tk, HK, 64, generator=g)
    v = torch.randn(B, Tk, HK, 64, generator=g)
    idx = torch.stack([torch.stack([torch.randperm(M, generator=g)[:S] for _ in range(HK)]) for _ in range(Tq)])
    idx = idx.unsqueeze(0)                    # (B, Tq, HK, S)
    w = None
    if mode == 2:
        w = torch.rand(B, Tq, HK, S, generator=g) + 0.05
    elif mode in (0, 3):
        w = torch.softmax(torch.randn(B, Tq, S, generator=g), -1)
    dO = torch.randn(B, Tq, HQ, 64, generator=g)
    scale = 0.125
    # the reference over keys padded to M * BS with masked keys: zero keys would still take
    # weight, so the padded rows get a large negative logit through -1e9 keys along one query dim
    rq, rk, rv = (t.to(dtype).double().requires_grad_(True) for t in (q, k, v))
    pad = M * BS - Tk
    kp = torch.cat([rk, torch.zeros(B, pad, HK, 64, dtype=torch.float64)], 1) if pad else rk
    vp = torch.cat([rv, torch.zeros(B, pad, HK, 64, dtype=torch.float64)], 1) if pad else rv
    rw = None if w is None else w.double().requires_grad_(True)
    if pad:
        # a query that selects the partial block sees only its Tk - (M - 1) BS real keys: give the
        # padding keys a logit of -inf by an extra query dimension (q . k_pad = -1e30)
        qx = torch.cat([rq, torch.ones(B, Tq, HQ, 1, dtype=torch.float64)], -1)
        kx = torch.cat([kp, torch.zeros(B, M * BS, HK, 1, dtype=torch.float64)], -1)
        kx = kx.clone()
        kx[:, Tk:, :, 64] = -1e30
        vx = torch.cat([vp, torch.zeros(B, M * BS, HK, 1, dtype=torch.float64)], -1)
    else:
        qx, kx, vx = rq, kp, vp
    f = REF[mode]
    ref = f(qx, kx, vx, idx, BS, scale) if mode == 1 else f(qx, kx, vx, idx, rw, BS, scale)
    ref = ref[..., :64]
    (ref * dO.to(dtype).double()).sum().backward()
    gq, gk, gv = (t.to(dev, dtype).requires_grad_(True) for t in (q, k, v))
    gw = None if w is None else w.to(dev).requires_grad_(True)
    kw = dict(softmax_scale=scale, disable_causal_mask=True)
    idx_d = idx.to(dev, torch.int32)
    if mode == 0:
        out = SA.FSA_topk_sparse_attention_weighted_bthd(gq, gk, gv, idx_d, gw, BS, **kw)
    elif mode == 3:
        out = SA.FSA_topk_sparse_attention_weighted_joint_bias_bthd(gq, gk, gv, idx_d, gw, BS, **kw)
    else:
        out = SA.FSA_topk_sparse_attention_bthd(gq, gk, gv, idx_d, BS, block_weights_bths=gw, **kw)
    assert out.dtype == dtype
    (out.float() * dO.to(dev)).sum().backward()
    chk = torch.bfloat16 if dtype == torch.float16 else dtype
    assert_parity(out, ref, chk, "out")
    assert_parity(gq.grad, rq.grad, chk, "dq")
    assert_parity(gk.grad, rk.grad, chk, "dk")
    assert_parity(gv.grad, rv.grad, chk, "dv")
    if w is not None:
        assert_parity(gw.grad, rw.grad, chk, "dw")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("weighted,version,shape", [(True, "v4", "dense"), (False, "v2", "dense"),
                                                    (True, "v5", "dense"), (True, "v4", "sparse"),
                                                    (False, "v2", "dense128"), (True, "v5", "dense128")])
def test_token_layer_matches_oracle(gpu_device, dtype, weighted, version, shape):
    """MemoryCrossAttention's token-routing path (shared dense + routed MoE) vs the oracle's
    token_memory_layer, including gradients of h, the bank and every projection.  "sparse":
    65 chapters, 4 tokens, k=2, so most routed chapters go unselected and their bank-gradient
    rows must come out exactly zero (the dK / dV rows are not pre-zeroed: the blocks no token
    selected are zeroed by moc_sparse_zero_untouched)."""
    print(f"token layer dtype={dtype} weighted={weighted} version={version} shape={shape}", flush=True)
    from memory_amd.memory_attention import MemoryCrossAttention
    from memory_amd.model import TokenRoutedMemoryLayer
    dev = gpu_device
    g = gen(55)
    B, Lq, d, H, C, T, S, k = {"dense": (2, 48, 128, 2, 9, 64, 1, 3), "sparse": (1, 4, 128, 2, 65, 64, 1, 2),
                               "dense128": (2, 48, 128, 2, 7, 128, 1, 3)}[shape]
    h = torch.randn(B, Lq, d, generator=g)
    bank = torch.randn(C * T, d, generator=g)
    Wr = torch.randn(C, d, generator=g) * 0.3
    br = torch.zeros(C)
    Wq, Wk, Wv, Wo = (torch.randn(d, d, generator=g) / d ** 0.5 for _ in range(4))
    layer = TokenRoutedMemoryLayer(d, H, C, T, k, num_shared_chapters=S, routed_scaling_factor=2.5,
                                   weighted=weighted, kernel_version=version, wo_init_zero=False)
    with torch.no_grad():
        layer.router.router.weight.copy_(Wr)
        layer.router.router.bias.copy_(br)
        for lin, W in zip((layer.memory_attn.q_proj, layer.memory_attn.k_proj, layer.memory_attn.v_proj,
                           layer.memory_attn.o_proj), (Wq, Wk, Wv, Wo)):
            lin.weight.copy_(W)
    layer = layer.to(dev)
    for m in (layer.memory_attn.q_proj, layer.memory_attn.k_proj, layer.memory_attn.v_proj, layer.memory_attn.o_proj):
        m.to(dtype)
    hg = h.to(dev, dtype).requires_grad_(True)
    bg = bank.to(dev, dtype).requires_grad_(True)
    out, _ = layer(hg, bg, return_losses=False)
    dO = torch.randn(out.shape, generator=gen(56))
    (out.float() * dO.to(dev)).sum().backward()

    leaves = [t.double().clone().requires_grad_(True) for t in (h, bank, Wr, br, Wq, Wk, Wv, Wo)]
    if dtype != torch.float32:
        # bf16 activations: the router GEMM rounds its weight to bf16 too (fp32 bias and logits)
        for i in (0, 1, 2, 4, 5, 6, 7):
            leaves[i] = leaves[i].detach().to(dtype).double().requires_grad_(True)
    if version == "v5" and weighted:
        ref = _token_layer_v5(*leaves, H=H, C=C, T=T, S=S, top_k=k)
    else:
        ref = O.token_memory_layer(*leaves, H=H, HK=H, C=C, T=T, S=S, top_k=k, routed_scale=2.5, weighted=weighted)
    (ref * dO.double()).sum().backward()
    assert_parity(out, ref, dtype, "out")
    names = ["dh", "dbank", "dWr", "dbr", "dWq", "dWk", "dWv", "dWo"]
    got = [hg.grad, bg.grad, layer.router.router.weight.grad, layer.router.router.bias.grad,
           layer.memory_attn.q_proj.weight.grad, layer.memory_attn.k_proj.weight.grad,
           layer.memory_attn.v_proj.weight.grad, layer.memory_attn.o_proj.weight.grad]
    for n, gr, r in zip(names, got, leaves):
        if r.grad is None or (not weighted and n in ("dWr", "dbr")):
            continue
        assert_parity(gr, r.grad, dtype, n)
    if shape == "sparse":
        idx, _, _ = layer.router.route_token_level(hg.detach(), return_losses=False, exclude_prefix_chapters=S)
        sel = torch.zeros(C, dtype=torch.bool)
        sel[:S] = True
        sel[idx.reshape(-1).cpu().long()] = True
        assert int((~sel).sum()) >= C // 2
        unsel = (~sel).repeat_interleave(T)
        assert int(torch.count_nonzero(bg.grad.cpu()[unsel])) == 0, "unselected chapters' bank rows must be zero"


def _token_layer_v5(h, bank, Wr, br, Wq, Wk, Wv, Wo, *, H, C, T, S, top_k):
    """Token layer with the v5 joint log-bias combine for the routed branch (the reference
    dispatches to kernel_v5 for weighted routing when the kernel version is v5)."""
    logits = O.linear(h, Wr, br)
    idx, w, _ = O.route_token_level(logits, top_k, S)
    B, Lq, d = h.shape
    shared = O.cross_attention(h, bank[:S * T], Wq, Wk, Wv, None, H, H, return_preproj=True)
    q, k, v = O.compute_qkv(h, bank[S * T:], Wq, Wk, Wv, H, H)
    idx4 = (idx - S).unsqueeze(2).expand(B, Lq, H, top_k)
    r = O.sparse_attention_joint_bias(q, k, v, idx4, w, T, q.shape[-1] ** -0.5)
    return O.linear(shared + r.reshape(B, Lq, -1) * 2.5, Wo)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hk0,nhk", [(0, 3), (1, 1)])
def test_zero_untouched_blocks(gpu_device, dtype, hk0, nhk):
    """moc_sparse_zero_untouched: the (chapter, kv head) blocks of dK / dV (rows layout) whose
    chapter the plan does not hold are zeroed, every other element is left as it was."""
    print(f"zero untouched {dtype} hk0={hk0} nhk={nhk}", flush=True)
    from memory_amd import _lib, ops
    C, HK, KV = 9, 3, 3 * 64
    chap = torch.tensor([4, 0, 4, 7, -1, 2], dtype=torch.int32, device=gpu_device)   # -1: skipped edge
    plan = ops.chapter_plan(chap, C)
    g = torch.Generator().manual_seed(3)
    dkv = (torch.randn(C * 64, 2 * KV, generator=g) + 5).to(dtype).to(gpu_device)
    before = dkv.clone()
    mark = torch.empty(C, dtype=torch.int32, device=gpu_device)
    es = dkv.element_size()
    _lib.call("moc_sparse_zero_untouched", _lib.dtype_code(dtype), dkv.data_ptr(), dkv.data_ptr() + KV * es,
              64 * 2 * KV, 64, 2 * KV, C, hk0, nhk, plan.uniq.data_ptr(), plan.n_uniq.data_ptr(), plan.max_u,
              mark.data_ptr(), _lib.stream_ptr(gpu_device))
    torch.cuda.synchronize()
    got, ref = dkv.cpu().view(C, 64, 2, HK, 64), before.cpu().view(C, 64, 2, HK, 64).clone()
    for c in range(C):
        if c not in (0, 2, 4, 7):
            ref[c, :, :, hk0:hk0 + nhk, :] = 0
    assert torch.equal(got, ref)


def test_token_path_moe_combine_needs_64_row_chapters(gpu_device):
    """The per-chapter MoE combine (v1-v4 with weights) keeps 64-row chapters: a longer chapter
    would split its softmax over sub-blocks, so it raises before any launch; the joint combines
    take any multiple of 64, and other lengths raise."""
    from memory_amd import sparse_attention as SA
    dev = gpu_device
    q = torch.zeros(1, 4, 2, 64, device=dev, dtype=torch.bfloat16)
    mem = torch.zeros(256, 128, device=dev, dtype=torch.bfloat16)
    w = torch.zeros(128, 128, device=dev, dtype=torch.bfloat16)
    idx = torch.zeros(1, 4, 1, device=dev, dtype=torch.int32)
    cw = torch.ones(1, 4, 1, device=dev)
    with pytest.raises(NotImplementedError, match="64-row chapters"):
        SA.token_routed_attention(q, mem, w, w, idx, cw, tokens_per_chapter=128, version="v4")
    with pytest.raises(ValueError, match="multiple of 64"):
        SA.token_routed_attention(q, mem, w, w, idx, None, tokens_per_chapter=96)


def _varlen_row_ref(mode, q, k, v, blocks, w, nb, BS, scale, HK):
    """One query row of the FSA modes over its own sequence's keys, straight from the
    definitions (float64): q (HQ, D); k, v (Nk_seq, HK, D); blocks (HK, S) local block ids, ids
    outside [0, nb) skipped; w: (HK, S) block weights (mode 2), (S,) chapter weights (0, 3)."""
    HQ = q.shape[0]
    G = HQ // HK
    outs = []
    for h in range(HQ):
        hk = h // G
        ids = [int(b) for b in blocks[hk]]
        if mode == 0:
            o = torch.zeros_like(q[h])
            for s_, b in enumerate(ids):
                if 0 <= b < nb:
                    kb, vb = k[b * BS:(b + 1) * BS, hk], v[b * BS:(b + 1) * BS, hk]
                    o = o + w[s_] * torch.softmax(scale * kb @ q[h], 0) @ vb
            outs.append(o)
            continue
        ks, vs, bias = [], [], []
        for s_, b in enumerate(ids):
            if 0 <= b < nb:
                ks.append(k[b * BS:(b + 1) * BS, hk])
                vs.append(v[b * BS:(b + 1) * BS, hk])
                if mode == 2:
                    bias.append(torch.log(w[hk, s_]).expand(BS))
                elif mode == 3:
                    bias.append(torch.log(torch.clamp(w[s_], min=1e-20)).expand(BS))
        kk, vv = torch.cat(ks), torch.cat(vs)
        z = scale * kk @ q[h]
        if bias:
            z = z + torch.cat(bias)
        outs.append(torch.softmax(z, 0) @ vv)
    return torch.stack(outs)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode,BS", [(1, 64), (2, 64), (0, 64), (3, 64), (1, 128), (0, 128), (3, 128)])
def test_fsa_varlen(gpu_device, dtype, mode, BS):
    """Packed variable-length inputs (cu_seqlens_q / cu_seqlens_k, kernel_v2.py:3181-3330): three
    sequences of 5, 17 and 9 queries over 128, 384 and 256 keys in one batch row, block ids local
    to each query's sequence; the first sequence names one block id past its keys in every row
    (skipped: out of the joint softmax, no contribution to the MoE combine).  Against the
    definitions evaluated row by row on each sequence alone (float64), gradients included."""
    print(f"fsa varlen mode={mode} BS={BS} dtype={dtype}", flush=True)
    from memory_amd import sparse_attention as SA
    dev = gpu_device
    g = gen(301 + mode + BS)
    HQ, HK, S, D = 4, 2, 2, 64
    lq, lk = [5, 17, 9], [128, 384, 256]
    cq = torch.tensor([0, 5, 22, 31], dtype=torch.int32)
    ck = torch.tensor([0, 128, 512, 768], dtype=torch.int32)
    Nq, Nk = 31, 768
    q = torch.randn(1, Nq, HQ, D, generator=g)
    k = torch.randn(1, Nk, HK, D, generator=g)
    v = torch.randn(1, Nk, HK, D, generator=g)
    idx = torch.zeros(1, Nq, HK, S, dtype=torch.long)
    for s_, (a, n, nk) in enumerate(zip(cq[:-1].tolist(), lq, lk)):
        nb = nk // BS
        for r in range(a, a + n):
            for h in range(HK):
                if s_ == 0:      # one valid block (< nb) and one id past the sequence
                    idx[0, r, h] = torch.tensor([int(torch.randint(nb, (1,), generator=g)), nb + r % 2])
                else:
                    idx[0, r, h] = torch.randperm(nb, generator=g)[:S]
    w = None
    if mode == 2:
        w = torch.rand(1, Nq, HK, S, generator=g) + 0.05
    elif mode in (0, 3):
        w = torch.softmax(torch.randn(1, Nq, S, generator=g), -1)
    dO = torch.randn(1, Nq, HQ, D, generator=g)
    scale = 0.125
    rq, rk, rv = (t.to(dtype).double().requires_grad_(True) for t in (q, k, v))
    rw = None if w is None else w.double().requires_grad_(True)
    rows = []
    for a, n, b0, nk in zip(cq[:-1].tolist(), lq, ck[:-1].tolist(), lk):
        for r in range(a, a + n):
            rows.append(_varlen_row_ref(mode, rq[0, r], rk[0, b0:b0 + nk], rv[0, b0:b0 + nk], idx[0, r],
                                        None if rw is None else rw[0, r], nk // BS, BS, scale, HK))
    ref = torch.stack(rows).unsqueeze(0)
    (ref * dO.to(dtype).double()).sum().backward()
    gq, gk, gv = (t.to(dev, dtype).requires_grad_(True) for t in (q, k, v))
    gw = None if w is None else w.to(dev).requires_grad_(True)
    kw = dict(softmax_scale=scale, disable_causal_mask=True, cu_seqlens_q=cq.to(dev), cu_seqlens_k=ck.to(dev))
    idx_d = idx.to(dev, torch.int32)
    if mode == 0:
        out = SA.FSA_topk_sparse_attention_weighted_bthd(gq, gk, gv, idx_d, gw, BS, **kw)
    elif mode == 3:
        out = SA.FSA_topk_sparse_attention_weighted_joint_bias_bthd(gq, gk, gv, idx_d, gw, BS, **kw)
    else:
        out = SA.FSA_topk_sparse_attention_bthd(gq, gk, gv, idx_d, BS, block_weights_bths=gw, **kw)
    (out.float() * dO.to(dev)).sum().backward()
    assert_parity(out, ref, dtype, "out")
    assert_parity(gq.grad, rq.grad, dtype, "dq")
    assert_parity(gk.grad, rk.grad, dtype, "dk")
    assert_parity(gv.grad, rv.grad, dtype, "dv")
    if w is not None:
        assert_parity(gw.grad, rw.grad, dtype, "dw")


def test_fsa_varlen_rejects_unaligned_keys(gpu_device):
    from memory_amd import sparse_attention as SA
    dev = gpu_device
    q = torch.randn(1, 4, 2, 64, device=dev)
    k = torch.randn(1, 192, 2, 64, device=dev)
    idx = torch.zeros(1, 4, 2, 1, dtype=torch.int32, device=dev)
    cq = torch.tensor([0, 2, 4], dtype=torch.int32, device=dev)
    with pytest.raises(NotImplementedError, match="boundary"):
        SA.FSA_topk_sparse_attention_bthd(q, k, k, idx, 64, cu_seqlens_q=cq,
                                          cu_seqlens_k=torch.tensor([0, 96, 192], dtype=torch.int32, device=dev),
                                          disable_causal_mask=True)
    with pytest.raises(ValueError, match="together"):
        SA.FSA_topk_sparse_attention_bthd(q, k, k, idx, 64, cu_seqlens_q=cq, disable_causal_mask=True)
