"""GPU parity of the forward kernels (router, plan, gather+K/V projection,
routed attention) against the CPU oracle on seeded inputs.

Tolerances: integer/index outputs bit-exact; fp32 within 1e-4 relative;
bf16 within 2e-2 relative max error (fp32 accumulation)."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from helpers import assert_parity, assert_rel, gen

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(gpu_device):
    from memory_amd import _lib
    _lib.lib()
    return gpu_device


def _ops():
    from memory_amd import ops
    return ops


# ------------------------------------------------------------------ router top-k

@pytest.mark.parametrize("R,C,S,k", [(8, 4097, 1, 64), (3, 33, 1, 4), (5, 33, 1, 32), (4, 50, 0, 7),
                                     (2, 1500, 3, 1), (6, 300, 2, 298), (100, 4097, 1, 16), (70, 257, 0, 40)])
def test_router_topk_matches_oracle(dev, R, C, S, k):
    print(f"router_topk R={R} C={C} S={S} k={k}", flush=True)
    logits = torch.randn(R, C, generator=gen(R * 1000 + C))
    idx, w = _ops().router_topk(logits.to(dev), k, S)
    ri, rw, _ = O.route_sequence(logits, k, S, select_by="logits")
    assert torch.equal(idx.cpu().long(), ri)
    assert_rel(w.cpu(), rw, 1e-5, "weights")


def test_router_topk_ties_lower_index_first(dev):
    g = gen(7)
    logits = torch.randint(-3, 3, (6, 257), generator=g).float()   # ~43 copies of each value
    idx, w = _ops().router_topk(logits.to(dev), 40, 1)
    ri = O.topk_desc_numpy(np.where(np.arange(257)[None, :] < 1, -np.inf, logits.numpy()), 40)
    assert np.array_equal(idx.cpu().numpy(), ri)
    _, rw, _ = O.route_sequence(logits, 40, 1)
    assert_rel(w.cpu(), rw, 1e-5, "tie weights")


@pytest.mark.parametrize("R", [2, 70])   # 1024- and 256-thread workgroups
@pytest.mark.parametrize("pattern", ["all_equal", "plateau", "plateau_low", "two_values"])
def test_router_topk_degenerate_rows(dev, R, pattern):
    """Rows the value-bin selection does not resolve by itself: every selectable logit equal
    (the k lowest ids), and a plateau of thousands of equal logits at the boundary (more than
    the boundary bin's direct ranking takes: the radix path), with ties to the lower id."""
    C, S, k = 4097, 1, 64
    g = gen(31)
    z = torch.zeros(R, C)
    if pattern == "plateau":          # 20 larger logits, one smaller, ~4,000 tied at the boundary
        z[:, torch.randperm(C, generator=g)[:20]] = 1.0
        z[:, 7] = -1.0
    elif pattern == "plateau_low":    # the plateau is the top: ties decide every slot
        z[:, torch.randperm(C, generator=g)[:30]] = -2.0
    elif pattern == "two_values":     # half the row at each of two values, k inside the upper half
        z[:, ::2] = 0.5
    z[:, 0] = 3.0                     # the shared prefix is excluded whatever its value
    print(f"router_topk degenerate R={R} pattern={pattern}", flush=True)
    idx, w = _ops().router_topk(z.to(dev), k, S)
    ri = O.topk_desc_numpy(np.where(np.arange(C)[None, :] < S, -np.inf, z.numpy()), k)
    assert np.array_equal(idx.cpu().numpy(), ri)
    _, rw, _ = O.route_sequence(z, k, S)
    assert_rel(w.cpu(), rw, 1e-5, "weights")


@pytest.mark.parametrize("R,C,S,k", [(4, 97, 1, 8), (80, 130, 2, 5), (3, 4097, 1, 64)])
def test_router_topk_backward_matches_autograd(dev, R, C, S, k):
    print(f"router_topk_bwd R={R} C={C} S={S} k={k}", flush=True)
    logits = torch.randn(R, C, generator=gen(11), dtype=torch.float64)
    dw = torch.randn(R, k, generator=gen(12), dtype=torch.float64)
    z = logits.clone().requires_grad_(True)
    ri, rw, _ = O.route_sequence(z, k, S, select_by="logits")
    (rw * dw).sum().backward()
    zg = logits.float().to(dev).requires_grad_(True)
    idx, w = _ops().router_topk(zg, k, S)
    (w * dw.float().to(dev)).sum().backward()
    assert torch.equal(idx.cpu().long(), ri)
    assert_rel(zg.grad.cpu(), z.grad, 1e-4, "dlogits")
    assert_parity(zg.grad.cpu(), z.grad, torch.float32, "dlogits")


def test_prepend_forward_backward(dev):
    R, k, S, s = 5, 6, 2, 2.5
    w = torch.rand(R, k, generator=gen(13), dtype=torch.float64)
    w = w / w.sum(-1, keepdim=True)
    idx = torch.randint(S, 40, (R, k), generator=gen(14))
    domega = torch.randn(R, S + k, generator=gen(15), dtype=torch.float64)
    wr = w.clone().requires_grad_(True)
    ci, cw = O.prepend_shared_chapters(idx, wr, num_chapters=40, num_shared_chapters=S, routed_scaling_factor=s)
    (cw * domega).sum().backward()
    wg = w.float().to(dev).requires_grad_(True)
    i2, w2 = _ops().prepend_shared(idx.to(dev), wg, S, s)
    (w2 * domega.float().to(dev)).sum().backward()
    assert torch.equal(i2.cpu().long(), ci)
    assert_rel(w2.cpu(), cw, 1e-6, "omega")
    assert_rel(wg.grad.cpu(), wr.grad, 1e-5, "dw")


@pytest.mark.parametrize("B,Lq,d,C", [(3, 37, 128, 65), (20, 70, 64, 33), (8, 1024, 768, 4097), (2, 33, 100, 17)])
def test_router_pool_and_linear(dev, B, Lq, d, C):
    print(f"router pool+linear B={B} L={Lq} d={d} C={C}", flush=True)
    h = torch.randn(B, Lq, d, generator=gen(16))
    W = torch.randn(C, d, generator=gen(17)) * 0.05
    b = torch.randn(C, generator=gen(18)) * 0.1
    coef = O.rolling_pool_coefficients(Lq, 5).float()
    for cf, ref_pool in ((None, O.sequence_pool(h.double())),
                         (coef, O.sequence_pool(h.double(), "sequence-rolling", 5))):
        hg = h.to(dev).requires_grad_(True)
        Wg = W.to(dev).requires_grad_(True)
        bg = b.to(dev).requires_grad_(True)
        pooled = _ops().router_pool(hg, None if cf is None else cf.to(dev))
        z = _ops().router_linear(pooled, Wg, bg)
        assert_rel(pooled.cpu(), ref_pool, 1e-5, "pooled")
        hr = h.double().requires_grad_(True)
        Wr = W.double().requires_grad_(True)
        br = b.double().requires_grad_(True)
        pr = O.sequence_pool(hr) if cf is None else O.sequence_pool(hr, "sequence-rolling", 5)
        zr = O.linear(pr, Wr, br)
        assert_rel(z.cpu(), zr, 1e-5, "logits")
        dz = torch.randn(B, C, generator=gen(19), dtype=torch.float64)
        (z * dz.float().to(dev)).sum().backward()
        (zr * dz).sum().backward()
        assert_rel(hg.grad.cpu(), hr.grad, 1e-5, "dh")
        assert_rel(Wg.grad.cpu(), Wr.grad, 1e-5, "dW")
        assert_rel(bg.grad.cpu(), br.grad, 1e-5, "db")
        for n, a, r in (("logits", z, zr), ("dh", hg.grad, hr.grad), ("dW", Wg.grad, Wr.grad), ("db", bg.grad, br.grad)):
            assert_parity(a.detach().cpu(), r.detach(), torch.float32, n)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("R,C", [(8192, 4097), (5, 3), (1000, 64)])
def test_col_sum(dev, dtype, R, C):
    """Column sums on the pooling kernels (router bias gradient of the token path)."""
    x = torch.randn(R, C, generator=gen(R + C)).to(dtype)
    got = _ops().col_sum(x.to(dev))
    assert_rel(got.cpu(), x.double().sum(0), 1e-5, "column sums")


# ------------------------------------------------------------------ chapter plan

@pytest.mark.parametrize("B,NS,C", [(8, 65, 4097), (2, 5, 33), (64, 65, 4097), (3, 7, 5), (300, 16, 4096),
                                    (16, 64, 300), (4, 20, 10000), (2048, 16, 33), (8192, 16, 4096)])
def test_chapter_plan_matches_numpy(dev, B, NS, C):
    g = np.random.default_rng(B * NS + C)
    chap = np.stack([g.choice(C, size=NS, replace=NS > C) for _ in range(B)]).astype(np.int32)
    chap[:, 0] = 0
    plan = _ops().chapter_plan(torch.from_numpy(chap).to(dev), C)
    n_u, n_bad = plan.n_uniq.cpu().tolist()
    flat = chap.reshape(-1)
    uniq = np.unique(flat)
    assert n_bad == 0 and n_u == len(uniq)
    assert np.array_equal(plan.uniq.cpu().numpy()[:n_u], uniq)
    assert np.array_equal(plan.edge_u.cpu().numpy(), np.searchsorted(uniq, flat))
    order = np.lexsort((np.arange(flat.size), flat))          # stable by (chapter, edge)
    assert np.array_equal(plan.csr_edge.cpu().numpy(), order)
    off = np.searchsorted(flat[order], uniq)
    assert np.array_equal(plan.csr_off.cpu().numpy()[:n_u], off)
    assert plan.csr_off.cpu().numpy()[n_u] == flat.size


def test_chapter_plan_skips_out_of_range(dev):
    chap = torch.tensor([[0, 3, 9, -1], [3, 12, 2, 9]], dtype=torch.int32)
    plan = _ops().chapter_plan(chap.to(dev), 10)
    n_u, n_bad = plan.n_uniq.cpu().tolist()
    assert (n_u, n_bad) == (4, 2)
    assert plan.uniq.cpu().tolist()[:4] == [0, 2, 3, 9]
    assert plan.edge_u.cpu().tolist() == [0, 2, 3, -1, 2, -1, 1, 3]
    assert plan.csr_off.cpu().tolist()[:5] == [0, 1, 2, 4, 6]
    assert plan.csr_edge.cpu().tolist()[:6] == [0, 6, 1, 4, 2, 7]


def test_chapter_plan_general_path_skips_out_of_range(dev):
    """More than 1,024 edges (the multi-block path): ids outside [0, C) are skipped, the rest
    planned as the stable (chapter, edge) order."""
    g = np.random.default_rng(7)
    C = 50
    chap = g.integers(-3, C + 3, size=(100, 30)).astype(np.int32)
    plan = _ops().chapter_plan(torch.from_numpy(chap).to(dev), C)
    flat = chap.reshape(-1)
    ok = (flat >= 0) & (flat < C)
    n_u, n_bad = plan.n_uniq.cpu().tolist()
    uniq = np.unique(flat[ok])
    assert (n_u, n_bad) == (len(uniq), int((~ok).sum()))
    assert np.array_equal(plan.uniq.cpu().numpy()[:n_u], uniq)
    eu = plan.edge_u.cpu().numpy()
    assert np.array_equal(eu[ok], np.searchsorted(uniq, flat[ok])) and (eu[~ok] == -1).all()
    idx = np.arange(flat.size)[ok]
    order = idx[np.lexsort((idx, flat[ok]))]
    assert np.array_equal(plan.csr_edge.cpu().numpy()[:ok.sum()], order)


@pytest.mark.parametrize("C", [1, 300, 4097])
def test_identity_plan_equals_plan_of_arange(dev, C):
    ops = _ops()
    ref = ops.chapter_plan(torch.arange(C, dtype=torch.int32, device=dev), C)
    got = ops.identity_plan(C, dev)
    assert (got.max_u, got.num_chapters) == (ref.max_u, ref.num_chapters)
    for name in ("uniq", "n_uniq", "edge_u", "csr_off", "csr_edge"):
        assert torch.equal(getattr(got, name).cpu(), getattr(ref, name).cpu()), name


# --------------------------------------------------- gather + K/V projection

@pytest.mark.parametrize("dtype,bank_dtype,norm", [(torch.float32, torch.float32, None),
                                                    (torch.float32, torch.float32, "rms"),
                                                    (torch.float32, torch.float32, "layernorm"),
                                                    (torch.bfloat16, torch.bfloat16, None),
                                                    (torch.bfloat16, torch.float32, "rms")])
def test_kv_project_matches_reference(dev, dtype, bank_dtype, norm):
    ops = _ops()
    C, T, d, HK, Dh = 40, 64, 256, 2, 64
    bank = torch.randn(C * T, d, generator=gen(20))
    wk = torch.randn(HK * Dh, d, generator=gen(21)) / d ** 0.5
    wv = torch.randn(HK * Dh, d, generator=gen(22)) / d ** 0.5
    chap = torch.tensor([[0, 7, 3, 39], [0, 3, 11, 25], [0, 39, 38, 1]], dtype=torch.int32)
    plan = ops.chapter_plan(chap.to(dev), C)
    bg = bank.to(dev, bank_dtype)
    code = ops.norm_code(norm)
    mean = rstd = None
    if code:
        mean, rstd = ops.row_stats(bg, plan, T, code, 1e-5)
    wkv = torch.cat([wk, wv]).to(dev, dtype)
    kt, vt, ktt, vtt = ops.kv_project(bg, plan, T, wkv, HK, Dh, mean, rstd, dtype, ("k", "v", "kt", "vt"))
    n_u = int(plan.n_uniq[0])
    uniq = plan.uniq[:n_u].cpu().long()
    X, _ = O.gather_chapters(bank.to(bank_dtype).double(), uniq.view(1, -1), T)
    X = X[0]
    if norm == "rms":
        X = O.rms_norm(X, 1e-5)
    elif norm == "layernorm":
        X = F.layer_norm(X, (d,), eps=1e-5)
    Kr = (X @ wk.to(dtype).double().T).view(n_u, T, HK, Dh).permute(0, 2, 1, 3)
    Vr = (X @ wv.to(dtype).double().T).view(n_u, T, HK, Dh).permute(0, 2, 1, 3)
    assert_parity(kt[:n_u].cpu(), Kr, dtype, "K tiles")
    assert_parity(vt[:n_u].cpu(), Vr, dtype, "V tiles")
    # the transposed tiles are the same values, bit for bit, with the key axis in MFMA order
    # (within each 32-key group: key 4g + e at position 8g + e, key 16 + 4g + e at 8g + 4 + e)
    pos = torch.tensor([32 * (k // 32) + (8 * ((k % 16) // 4) + (k % 4) + (4 if k % 32 >= 16 else 0))
                        for k in range(T)])
    assert sorted(pos.tolist()) == list(range(T))
    assert torch.equal(ktt[:n_u][..., pos].transpose(-1, -2).cpu(), kt[:n_u].cpu())
    assert torch.equal(vtt[:n_u][..., pos].transpose(-1, -2).cpu(), vt[:n_u].cpu())


# --------------------------------------------------- routed attention forward

def _seq_case(seed, B, Lq, d, H, HK, C, T, S, k, scale_in=1.0):
    g = gen(seed)
    h = torch.randn(B, Lq, d, generator=g)
    bank = torch.randn(C * T, d, generator=g) * scale_in
    Wr = torch.randn(C, d, generator=g) * 0.02
    Dh = d // H
    Wq = torch.randn(H * Dh, d, generator=g) / d ** 0.5
    Wk = torch.randn(HK * Dh, d, generator=g) / d ** 0.5
    Wv = torch.randn(HK * Dh, d, generator=g) / d ** 0.5
    logits = torch.randn(B, C, generator=g) * 2.0
    idx, w, _ = O.route_sequence(logits, k, S)
    ci, cw = O.prepend_shared_chapters(idx, w, num_chapters=C, num_shared_chapters=S, routed_scaling_factor=2.5)
    return h, bank, Wq, Wk, Wv, ci, cw


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,Lq,H,HK,norm", [(2, 128, 4, 4, None), (2, 100, 4, 2, "rms"), (3, 257, 2, 1, None),
                                            (1, 1, 4, 4, "layernorm")])
def test_routed_attention_forward(dev, dtype, B, Lq, H, HK, norm):
    print(f"routed_attention fwd dtype={dtype} B={B} L={Lq} H={H} HK={HK} norm={norm}", flush=True)
    ops = _ops()
    d, C, T, S, k = H * 64, 33, 64, 1, 4
    h, bank, Wq, Wk, Wv, ci, cw = _seq_case(23, B, Lq, d, H, HK, C, T, S, k)
    q = (h @ Wq.T).view(B, Lq, H, 64)
    out = ops.routed_attention(q.to(dev, dtype), bank.to(dev, dtype), Wk.to(dev, dtype), Wv.to(dev, dtype),
                               cw.to(dev), ci.to(dev), num_chapters=C, tokens_per_chapter=T, norm_type=norm,
                               eps=1e-5, num_kv_heads=HK)
    hd, bd = h.double(), bank.to(dtype).double()
    mem, _ = O.gather_chapters(bd, ci, T)
    if norm:
        mem = O.normalize_shared_routed(mem, num_shared_chapters=S, tokens_per_chapter=T, norm_type=norm, eps=1e-5)
    mem = O.weight_memory(mem, cw.double(), T)
    qr = q.to(dtype).double()
    kr = (mem @ Wk.to(dtype).double().T).view(B, -1, HK, 64)
    vr = (mem @ Wv.to(dtype).double().T).view(B, -1, HK, 64)
    ref = O.attention(qr, kr, vr)
    assert_parity(out.cpu(), ref, dtype, "attention output")


@pytest.mark.parametrize("R,C,k,scale", [(8, 4097, 64, 1.0), (300, 257, 5, 3.0), (1, 33, 4, 1.0),
                                         (1024, 4097, 16, 0.5), (5, 16000, 3, 1.0), (40, 65, 0, 1.0),
                                         (7, 4608, 8, 1.0), (7, 4609, 8, 1.0)])
def test_router_losses_fused_match_oracle(dev, R, C, k, scale):
    """The fused router-loss kernels (router.py:197-260): the four losses and the gradient of a
    random combination of them w.r.t. the logits, against the oracle in float64."""
    print(f"router losses R={R} C={C} k={k}", flush=True)
    g = gen(R + C + k)
    logits = torch.randn(R, C, generator=g, dtype=torch.float64) * scale
    logits[0, : min(5, C)] += 6.0          # a peaked row (entropy / z-loss away from uniform)
    idx = torch.stack([torch.randperm(C, generator=g)[:k] for _ in range(R)]) if k else torch.empty(R, 0, dtype=torch.long)
    coef = torch.rand(4, generator=g, dtype=torch.float64) + 0.5
    lr = logits.clone().requires_grad_(True)
    ref = O.router_losses(lr, torch.softmax(lr, dim=-1), idx, C)
    names = ("load_balance", "auxiliary", "z_loss", "entropy")
    sum(coef[i] * ref[n] for i, n in enumerate(names)).backward()
    lg = logits.float().to(dev).requires_grad_(True)
    got = _ops().router_losses(lg, idx.to(dev), C)
    sum(float(coef[i]) * got[n] for i, n in enumerate(names)).backward()
    for n in names:
        assert_rel(got[n].reshape(1).cpu(), ref[n].reshape(1).detach(), 1e-5, n)
    assert_rel(lg.grad.cpu(), lr.grad, 1e-4, "dlogits")


@pytest.mark.parametrize("M,K,N,odt", [(1, 768, 768, torch.bfloat16), (64, 768, 768, torch.bfloat16),
                                       (65, 640, 48, torch.float32), (7, 128, 16, torch.bfloat16),
                                       (256, 2048, 1536, torch.float32), (200, 896, 256, torch.bfloat16)])
def test_linear_rows_matches_fp64(dev, M, K, N, odt):
    """The few-row x W^T kernel (decode q_proj / o_proj) against a float64 product of the same
    bf16 operands."""
    from memory_amd import ops
    g = gen(M + K + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g) * K ** -0.5).to(torch.bfloat16)
    y = torch.empty(M, N, device=dev, dtype=odt)
    from memory_amd import _lib as L
    xd, Wd = x.to(dev), W.to(dev)          # held: the kernel reads them after the call returns
    L.call("moc_linear_rows", L.ptr(xd), M, K, L.ptr(Wd), N, L.dtype_code(odt), L.ptr(y), L.stream_ptr(dev))
    torch.cuda.synchronize()
    ref = x.double() @ W.double().t()
    assert_rel(y.float().cpu(), ref, 1e-5 if odt == torch.float32 else 1e-2, "x W^T")
    # the product path dispatches few-row bf16 inputs here
    assert_rel(ops.linear(xd, Wd).float().cpu(), ref, 1e-2, "ops.linear")
