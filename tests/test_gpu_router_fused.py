"""The fused router kernels of the sequence-routed layer against the separate launches they
replace and against the oracle:

* moc_router_topk_prepend == moc_router_topk then moc_prepend_shared, bit for bit (ids,
  weights, prepended ids and omega), on the 1,024-thread (few rows) and 256-thread variants,
  with tied logits;
* moc_router_seq_bwd == (sum over kv heads of the d omega partials) -> moc_prepend_shared_bwd
  -> moc_router_topk_bwd (+ the incoming logit gradient), and against autograd of the oracle's
  route_sequence + prepend_shared_chapters (router.py:114-149, model.py:356-391) in fp64;
* moc_router_pool1 against the oracle's pooling (router.py:96-107 mean, :158-195 rolling);
* moc_rows_add_bcast against a torch broadcast add."""

import pytest
import torch

import oracle as O
from helpers import assert_rel
from memory_amd import _lib as L

pytestmark = pytest.mark.gpu


def _topk_prepend_both(logits, S, k, scale):
    dev = logits.device
    R, C = logits.shape
    i1 = torch.empty(R, k, device=dev, dtype=torch.int32)
    w1 = torch.empty(R, k, device=dev, dtype=torch.float32)
    L.call("moc_router_topk", L.ptr(logits), R, C, S, k, L.ptr(i1), L.ptr(w1), None, L.stream_ptr(dev))
    is1 = torch.empty(R, S + k, device=dev, dtype=torch.int32)
    om1 = torch.empty(R, S + k, device=dev, dtype=torch.float32)
    L.call("moc_prepend_shared", L.ptr(i1), L.ptr(w1), R, k, S, scale, L.ptr(is1), L.ptr(om1), L.stream_ptr(dev))
    i2 = torch.full((R, k), -7, device=dev, dtype=torch.int32)
    w2 = torch.full((R, k), -7.0, device=dev, dtype=torch.float32)
    is2 = torch.full((R, S + k), -7, device=dev, dtype=torch.int32)
    om2 = torch.full((R, S + k), -7.0, device=dev, dtype=torch.float32)
    L.call("moc_router_topk_prepend", L.ptr(logits), R, C, S, k, scale, L.ptr(i2), L.ptr(w2), L.ptr(is2),
           L.ptr(om2), L.stream_ptr(dev))
    torch.cuda.synchronize()
    return (i1, w1, is1, om1), (i2, w2, is2, om2)


@pytest.mark.parametrize("R,C,S,k", [(8, 4097, 1, 64), (3, 33, 1, 4), (100, 517, 3, 16), (2, 2048, 5, 1024 - 5)])
def test_topk_prepend_matches_separate_launches(gpu_device, R, C, S, k):
    print(f"topk+prepend R={R} C={C} S={S} k={k}", flush=True)
    g = torch.Generator().manual_seed(R * 7 + C)
    logits = torch.randn(R, C, generator=g) * 0.05
    logits[:, 5:40] = 0.01   # ties around the threshold
    logits = logits.to(gpu_device)
    a, b = _topk_prepend_both(logits, S, k, 2.5)
    for x, y, n in zip(a, b, ("idx", "w", "idx_star", "omega")):
        assert torch.equal(x, y), n


def _seq_bwd_both(logits, idx, w, dom_part, HK, S, k, scale, dz_in):
    dev = logits.device
    R, C = logits.shape
    NS = S + k
    st = L.stream_ptr(dev)
    domega = dom_part.view(R * NS, HK).double().sum(-1).float().view(R, NS).contiguous()
    dw = torch.empty(R, k, device=dev, dtype=torch.float32)
    L.call("moc_prepend_shared_bwd", L.ptr(w), L.ptr(domega), R, k, S, scale, L.ptr(dw), st)
    dz1 = torch.empty(R, C, device=dev, dtype=torch.float32)
    L.call("moc_router_topk_bwd", L.ptr(logits), L.ptr(idx), L.ptr(dw), R, C, S, k, L.ptr(dz1), st)
    if dz_in is not None:
        dz1 = dz1 + dz_in
    dz2 = torch.full((R, C), float("nan"), device=dev, dtype=torch.float32)
    L.call("moc_router_seq_bwd", L.ptr(logits), L.ptr(idx), L.ptr(w), L.ptr(dom_part), HK, R, C, S, k, scale,
           L.ptr(dz_in), L.ptr(dz2), st)
    torch.cuda.synchronize()
    return dz1, dz2


@pytest.mark.parametrize("R,C,S,k,HK,with_in", [(8, 4097, 1, 64, 12, True), (3, 33, 1, 4, 4, False),
                                                (100, 517, 3, 16, 2, True)])
def test_router_seq_bwd_matches_chain(gpu_device, R, C, S, k, HK, with_in):
    print(f"router_seq_bwd R={R} C={C} S={S} k={k} HK={HK} dz_in={with_in}", flush=True)
    dev = gpu_device
    g = torch.Generator().manual_seed(R + C + HK)
    logits = (torch.randn(R, C, generator=g) * 0.3).to(dev)
    idx = torch.empty(R, k, device=dev, dtype=torch.int32)
    w = torch.empty(R, k, device=dev, dtype=torch.float32)
    L.call("moc_router_topk", L.ptr(logits), R, C, S, k, L.ptr(idx), L.ptr(w), None, L.stream_ptr(dev))
    dom_part = torch.randn(R * (S + k), HK, generator=g).to(dev)
    dz_in = torch.randn(R, C, generator=g).to(dev) if with_in else None
    dz1, dz2 = _seq_bwd_both(logits, idx, w, dom_part, HK, S, k, 2.5, dz_in)
    assert torch.isfinite(dz2).all()
    assert_rel(dz2, dz1, 1e-5, "dlogits")

    # against autograd of the oracle (fp64): d/dlogits of sum(domega * omega) (+ dz_in . logits)
    z = logits.cpu().double().requires_grad_(True)
    sel, wo, _ = O.route_sequence(z, k, S)
    assert torch.equal(sel.to(torch.int32), idx.cpu())
    _, om = O.prepend_shared_chapters(sel, wo, num_chapters=C, num_shared_chapters=S, routed_scaling_factor=2.5)
    loss = (om * dom_part.cpu().double().view(R, S + k, HK).sum(-1)).sum()
    if dz_in is not None:
        loss = loss + (z * dz_in.cpu().double()).sum()
    loss.backward()
    assert_rel(dz2, z.grad, 1e-4, "dlogits vs oracle")


@pytest.mark.parametrize("B,Lq,d,rolling", [(8, 1024, 768, False), (3, 77, 256, True), (2, 5, 64, False)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_pool1_matches_oracle(gpu_device, B, Lq, d, rolling, dtype):
    print(f"pool1 B={B} L={Lq} d={d} rolling={rolling} {dtype}", flush=True)
    dev = gpu_device
    g = torch.Generator().manual_seed(B * Lq + d)
    h = torch.randn(B, Lq, d, generator=g).to(dtype)
    coef = None
    if rolling:
        from memory_amd.router import rolling_coefficients
        coef = rolling_coefficients(Lq, 16, dev)
        ref = O.sequence_pool(h.double(), strategy="sequence-rolling", window=16)
    else:
        ref = O.sequence_pool(h.double())
    hd = h.to(dev)
    out = torch.empty(B, d, device=dev, dtype=torch.float32)
    L.call("moc_router_pool1", L.ptr(hd), L.dtype_code(dtype), B, Lq, d, L.ptr(coef), L.ptr(out),
           L.stream_ptr(dev))
    assert_rel(out, ref, 1e-5, "pooled")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("with_coef", [False, True])
def test_rows_add_bcast(gpu_device, dtype, with_coef):
    dev = gpu_device
    g = torch.Generator().manual_seed(5)
    B, Lq, d = 3, 37, 264
    x = torch.randn(B, Lq, d, generator=g).to(dtype)
    v = torch.randn(B, d, generator=g)
    coef = torch.rand(Lq, generator=g) if with_coef else None
    ref = x.double() + v.double().unsqueeze(1) * (coef.double().view(1, Lq, 1) if with_coef else 0.25)
    xd = x.to(dev)
    vd = v.to(dev)
    cd = None if coef is None else coef.to(dev)
    L.call("moc_rows_add_bcast", L.ptr(xd), L.dtype_code(dtype), B, Lq, d, L.ptr(vd), L.ptr(cd), 0.25,
           L.stream_ptr(dev))
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-6
    assert_rel(xd, ref, tol, "x + v")


@pytest.mark.parametrize("R,C", [(8192, 4097), (100, 33), (65, 512)])
def test_logit_grad_pack(gpu_device, R, C):
    """moc_logit_grad_pack: the bf16 copy of the per-token router's logit gradient, padded with
    zero columns to a multiple of 256 (exactly torch's round-to-nearest conversion), and the bias
    gradient db = sum over rows (router.py:294's nn.Linear bias) against float64."""
    dev = gpu_device
    g = torch.Generator().manual_seed(R + C)
    dz = torch.randn(R, C, generator=g) * torch.rand(R, 1, generator=g) * 3
    Cp = (C + 255) // 256 * 256
    dzd = dz.to(dev)
    dzp = torch.full((R, Cp), float("nan"), device=dev, dtype=torch.bfloat16)
    db = torch.empty(C, device=dev)
    ws_bytes = L.query("moc_logit_grad_pack_workspace", R, C)
    ws = torch.empty(ws_bytes // 4, device=dev)
    L.call("moc_logit_grad_pack", L.ptr(dzd), R, C, Cp, L.ptr(dzp), L.ptr(db), L.ptr(ws), ws_bytes, L.stream_ptr(dev))
    got = dzp.cpu()
    assert torch.equal(got[:, :C], dz.to(torch.bfloat16)), "bf16 copy"
    assert (got[:, C:] == 0).all(), "padding columns must be zero"
    assert_rel(db.cpu(), dz.double().sum(0), 1e-5, "db")
    # without the bias gradient: only the copy
    dzp2 = torch.full((R, Cp), float("nan"), device=dev, dtype=torch.bfloat16)
    L.call("moc_logit_grad_pack", L.ptr(dzd), R, C, Cp, L.ptr(dzp2), None, None, 0, L.stream_ptr(dev))
    assert torch.equal(dzp2.cpu(), got)


@pytest.mark.parametrize("R,C,S,k,with_in", [(8192, 4097, 1, 16, False), (8192, 4097, 1, 16, True),
                                             (200, 300, 0, 5, True), (97, 4600, 3, 64, False)])
def test_topk_bwd_pack_matches_chain(gpu_device, R, C, S, k, with_in):
    """moc_router_topk_bwd_pack == moc_router_topk_bwd (+ the incoming logit gradient) then the
    bf16 copy: the padded bf16 rows bit for bit, the bias gradient (column sums) against float64
    sums of the chain's fp32 gradient; row counts that are not a multiple of the 32-row groups."""
    dev = gpu_device
    g = torch.Generator().manual_seed(R + C + k)
    logits = (torch.randn(R, C, generator=g) * 2).to(dev)
    idx = torch.empty(R, k, device=dev, dtype=torch.int32)
    w = torch.empty(R, k, device=dev, dtype=torch.float32)
    L.call("moc_router_topk", L.ptr(logits), R, C, S, k, L.ptr(idx), L.ptr(w), None, L.stream_ptr(dev))
    dw = torch.randn(R, k, generator=g).to(dev)
    dz_in = torch.randn(R, C, generator=g).to(dev) * 1e-3 if with_in else None
    ref = torch.empty(R, C, device=dev)
    L.call("moc_router_topk_bwd", L.ptr(logits), L.ptr(idx), L.ptr(dw), R, C, S, k, L.ptr(ref), L.stream_ptr(dev))
    if with_in:
        ref = ref + dz_in
    Cp = min((C + 255) // 256 * 256, 4608)
    dzp = torch.full((R, Cp), float("nan"), device=dev, dtype=torch.bfloat16)
    db = torch.empty(C, device=dev)
    ws_bytes = L.query("moc_router_topk_bwd_pack_workspace", R, C)
    ws = torch.empty(ws_bytes // 4, device=dev)
    L.call("moc_router_topk_bwd_pack", L.ptr(logits), L.ptr(idx), L.ptr(dw), R, C, S, k, L.ptr(dz_in), Cp, L.ptr(dzp),
           L.ptr(db), L.ptr(ws), ws_bytes, L.stream_ptr(dev))
    got = dzp.cpu()
    assert torch.equal(got[:, :C], ref.cpu().to(torch.bfloat16)), "bf16 logit gradient"
    assert (got[:, C:] == 0).all(), "padding columns must be zero"
    assert_rel(db.cpu(), ref.cpu().double().sum(0), 1e-5, "db")


@pytest.mark.parametrize("with_losses", [False, True])
def test_token_router_fused_gradients(gpu_device, with_losses):
    """The fused per-token router (ops.token_router: logits GEMM + top-k in one function, its
    backward through moc_router_topk_bwd_pack) against the two-function composition on the same
    inputs: logits, ids and weights equal; dx, dW and db within the bf16 / fp32 gates."""
    from memory_amd import ops
    from memory_amd.router import compute_router_losses
    from helpers import assert_parity
    dev = gpu_device
    g = torch.Generator().manual_seed(11 + with_losses)
    R, d, C, k, S = 1024, 256, 1025, 8, 1
    x0 = (torch.randn(R, d, generator=g)).to(dev, torch.bfloat16)
    W0 = (torch.randn(C, d, generator=g) * 0.05).to(dev)
    b0 = (torch.randn(C, generator=g) * 0.1).to(dev)
    dw = torch.randn(R, k, generator=g).to(dev)
    outs = []
    for fused in (True, False):
        x = x0.clone().requires_grad_(True)
        W = W0.clone().requires_grad_(True)
        b = b0.clone().requires_grad_(True)
        if fused:
            assert ops.token_router_fused_ok(x, C, k)
            logits, idx, w = ops._TokenRouter.apply(x, W, b, k, S)
        else:
            logits = ops.router_token_logits(x, W, b)
            idx, w = ops.router_topk(logits, k, S)
        loss = (w * dw).sum()
        if with_losses:
            losses = compute_router_losses(logits, None, idx, C)
            loss = loss + 0.3 * losses["load_balance"] + 0.01 * losses["z_loss"]
        loss.backward()
        outs.append((logits.detach(), idx, w.detach(), x.grad, W.grad, b.grad))
    (l1, i1, w1, dx1, dW1, db1), (l2, i2, w2, dx2, dW2, db2) = outs
    assert torch.equal(l1, l2) and torch.equal(i1, i2) and torch.equal(w1, w2)
    assert_parity(dx1, dx2.float(), torch.bfloat16, "dx")
    assert_parity(dW1, dW2, torch.float32, "dW")
    assert_parity(db1, db2, torch.float32, "db")
