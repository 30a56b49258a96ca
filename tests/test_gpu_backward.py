"""GPU parity of the routed-attention backward against autograd of the CPU
oracle (float64) on the same seeded inputs.

Gate (tests/helpers.py): fp32 every element within 1e-4 relative; bf16 max-abs 2e-2 (bf16
operands, fp32 accumulation).  Cases cover GQA, row
normalisation (rms / layernorm), ragged L, and chapters selected by several
sequences (the chapter-centric dK/dV accumulation across the batch)."""

import pytest
import torch

import oracle as O
from helpers import assert_parity, gen

pytestmark = pytest.mark.gpu


def _ref_grads(q, bank, Wk, Wv, ci, cw, dO, T, S, norm, HK):
    B, Lq, H, Dh = q.shape
    leaves = [t.detach().double().clone().requires_grad_(True) for t in (q, bank, Wk, Wv, cw)]
    qd, bd, wkd, wvd, cwd = leaves
    mem, _ = O.gather_chapters(bd, ci, T)
    if norm:
        mem = O.normalize_shared_routed(mem, num_shared_chapters=S, tokens_per_chapter=T, norm_type=norm, eps=1e-5)
    mem = O.weight_memory(mem, cwd, T)
    k = (mem @ wkd.T).view(B, -1, HK, Dh)
    v = (mem @ wvd.T).view(B, -1, HK, Dh)
    out = O.attention(qd, k, v)
    (out * dO.double()).sum().backward()
    return out.detach(), [t.grad for t in leaves]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,Lq,H,HK,C,k,norm,dup,zero_w", [
    (2, 128, 4, 4, 33, 4, None, False, False),
    (3, 100, 4, 2, 12, 5, "rms", True, False),
    (2, 130, 2, 1, 20, 3, "layernorm", True, False),
    (4, 64, 4, 4, 9, 8, None, True, False),
    (3, 96, 4, 2, 16, 6, None, True, True),
    (3, 96, 4, 2, 16, 6, None, True, "tiny"),
])
def test_routed_attention_backward(gpu_device, dtype, B, Lq, H, HK, C, k, norm, dup, zero_w):
    print(f"routed_attention bwd dtype={dtype} B={B} L={Lq} H={H} HK={HK} C={C} k={k} norm={norm} "
          f"zero_w={zero_w}", flush=True)
    from memory_amd import ops
    dev = gpu_device
    g = gen(100 + B + Lq)
    T, S, Dh = 64, 1, 64
    d = 128
    h = torch.randn(B, Lq, d, generator=g)
    bank = torch.randn(C * T, d, generator=g)
    Wq = torch.randn(H * Dh, d, generator=g) / d ** 0.5
    Wk = torch.randn(HK * Dh, d, generator=g) / d ** 0.5
    Wv = torch.randn(HK * Dh, d, generator=g) / d ** 0.5
    logits = torch.randn(B, C, generator=g) * 2
    if dup:   # make every sequence pick (mostly) the same chapters
        logits = logits[:1].expand(B, C) + 0.01 * torch.randn(B, C, generator=g)
    idx, w, _ = O.route_sequence(logits, k, S)
    ci, cw = O.prepend_shared_chapters(idx, w, num_chapters=C, num_shared_chapters=S, routed_scaling_factor=2.5)
    if zero_w == "tiny":
        # positive weights far below fp32 resolution (a denormal, and one whose square underflows):
        # outputs and gradients finite and equal to the oracle's
        cw = cw.clone()
        cw[:, 2] = 1e-39
        cw[0, 4] = 1e-30
        cw[1, 3] = 1e-20
    elif zero_w:
        # exact-zero chapter weights: keys / values vanish, d omega does not
        cw = cw.clone()
        cw[:, 2] = 0.0
        cw[0, 4] = 0.0
    q = (h @ Wq.T).view(B, Lq, H, Dh)
    dO = torch.randn(B, Lq, H, Dh, generator=g)

    qg = q.to(dev, dtype).requires_grad_(True)
    bg = bank.to(dev, dtype).requires_grad_(True)
    wkg = Wk.to(dev, dtype).requires_grad_(True)
    wvg = Wv.to(dev, dtype).requires_grad_(True)
    cwg = cw.to(dev).requires_grad_(True)
    out = ops.routed_attention(qg, bg, wkg, wvg, cwg, ci.to(dev), num_chapters=C, tokens_per_chapter=T,
                               norm_type=norm, eps=1e-5, num_kv_heads=HK)
    (out.float() * dO.to(dev)).sum().backward()

    rdt = lambda t: t.to(dtype)  # reference sees the same rounded inputs
    ref_out, (gq, gb, gk, gv, gw) = _ref_grads(rdt(q), rdt(bank), rdt(Wk), rdt(Wv), ci, cw, rdt(dO).float(), T, S,
                                               norm, HK)
    assert_parity(out, ref_out, dtype, "out")
    assert_parity(qg.grad, gq, dtype, "dq")
    assert_parity(wkg.grad, gk, dtype, "dWk")
    assert_parity(wvg.grad, gv, dtype, "dWv")
    assert_parity(bg.grad, gb, dtype, "dbank")
    assert_parity(cwg.grad, gw, dtype, "domega")
    for t, name in ((out, "out"), (qg.grad, "dq"), (bg.grad, "dbank"), (cwg.grad, "domega")):
        assert torch.isfinite(t.float()).all(), f"{name} not finite"
    # rows of chapters nobody selected get exactly zero gradient
    sel = torch.zeros(C, dtype=torch.bool)
    sel[ci.reshape(-1)] = True
    unsel = (~sel).repeat_interleave(T)
    assert torch.count_nonzero(bg.grad.cpu()[unsel]) == 0


@pytest.mark.parametrize("d,HK,C,nsel,bank_dtype,norm,out_dtype", [
    (768, 12, 60, 41, torch.bfloat16, None, torch.bfloat16),
    (128, 1, 20, 7, torch.bfloat16, "rms", torch.float32),
    (200, 2, 30, 12, torch.float32, "layernorm", torch.float32),
    (256, 4, 9, 9, torch.bfloat16, None, torch.float32),
])
def test_kv_weight_grad_kernel(gpu_device, d, HK, C, nsel, bank_dtype, norm, out_dtype):
    """dW = dkv^T norm(gather(bank)) from the split-row kernel against float64 on the same
    bf16-rounded operands (tolerance 2e-2 relative max error, fp32 accumulation)."""
    print(f"kv_wgrad d={d} HK={HK} C={C} nsel={nsel} bank={bank_dtype} norm={norm} out={out_dtype}", flush=True)
    from memory_amd import _lib as L
    from memory_amd import ops
    dev = gpu_device
    T, KV2 = 64, 2 * HK * 64
    g = gen(300 + d + HK)
    bank = torch.randn(C * T, d, generator=g)
    chap = torch.randperm(C, generator=g)[:nsel].to(torch.int32).view(1, -1)
    plan = ops.chapter_plan(chap.to(dev), C)
    bg = bank.to(dev, bank_dtype)
    code = ops.norm_code(norm)
    mean = rstd = None
    if code:
        mean, rstd = ops.row_stats(bg, plan, T, code, 1e-5)
    max_u = plan.max_u
    dkv = torch.randn(max_u * T, KV2, generator=g).to(torch.bfloat16)
    n_u = int(plan.n_uniq[0])
    dkv[n_u * T:] = 0
    ws = torch.empty(L.query("moc_kv_wgrad_workspace", KV2, d, max_u) // 4, device=dev, dtype=torch.float32)
    dw = torch.full((KV2, d), float("nan"), device=dev, dtype=out_dtype)
    dkv_d = dkv.to(dev)  # kept alive until the kernel has run
    L.call("moc_kv_wgrad", L.ptr(dkv_d), L.ptr(bg), L.dtype_code(bank_dtype), d, T, L.ptr(plan.uniq),
           L.ptr(plan.n_uniq), None, max_u, L.ptr(mean), L.ptr(rstd), KV2, L.ptr(ws), ws.numel() * 4,
           L.dtype_code(out_dtype), L.ptr(dw), L.stream_ptr(dev))
    uniq = plan.uniq[:n_u].cpu().long()
    X, _ = O.gather_chapters(bg.cpu().double(), uniq.view(1, -1), T)
    X = X[0]
    if norm == "rms":
        X = O.rms_norm(X, 1e-5)
    elif norm == "layernorm":
        X = torch.nn.functional.layer_norm(X, (d,), eps=1e-5)
    X = X.to(torch.bfloat16).double()  # the kernel feeds bf16 operands to the MFMA
    ref = dkv[:n_u * T].double().T @ X
    assert_parity(dw, ref, out_dtype, "dW")


@pytest.mark.parametrize("R,N,K,x_dtype,out_dtype", [
    (8192, 768, 768, torch.bfloat16, torch.bfloat16),
    (1000, 136, 200, torch.float32, torch.float32),
    (64, 512, 128, torch.bfloat16, torch.float32),
])
def test_linear_weight_grad_kernel(gpu_device, R, N, K, x_dtype, out_dtype):
    """dW = dy^T x of the dense projections (split-row kernel) against float64 on the same
    bf16-rounded operands, including a ragged row count (2e-2 relative max error)."""
    print(f"linear_wgrad R={R} N={N} K={K} x={x_dtype} out={out_dtype}", flush=True)
    from memory_amd import _lib as L
    dev = gpu_device
    g = gen(400 + R + N)
    dy = torch.randn(R, N, generator=g).to(torch.bfloat16)
    x = torch.randn(R, K, generator=g).to(x_dtype)
    ws = torch.empty(L.query("moc_linear_wgrad_workspace", R, N, K) // 4, device=dev, dtype=torch.float32)
    dw = torch.full((N, K), float("nan"), device=dev, dtype=out_dtype)
    dy_d, x_d = dy.to(dev), x.to(dev)  # kept alive until the kernel has run
    L.call("moc_linear_wgrad", L.ptr(dy_d), L.ptr(x_d), L.dtype_code(x_dtype), R, N, K, L.ptr(ws),
           ws.numel() * 4, L.dtype_code(out_dtype), L.ptr(dw), L.stream_ptr(dev))
    ref = dy.double().T @ x.to(torch.bfloat16).double()
    assert_parity(dw, ref, out_dtype, "dW")


@pytest.mark.parametrize("shape", [(3, 130, 256, 384), (3, 130, 256, 512), (8, 1024, 768, 768)])
def test_linear_autograd_matches_reference(gpu_device, shape):
    """ops.linear (q_proj / o_proj) gradients against float64 autograd, bf16 operands, with the
    weight gradient on the split-row kernel (384 outputs) and on the LDS-DMA kernel
    (256-multiples, over a row count that leaves a partial 64-row block, and at the c3 shape)."""
    from memory_amd import ops
    dev = gpu_device
    B, Lq, K, N = shape
    g = gen(77)
    x = torch.randn(B, Lq, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) / 16).to(torch.bfloat16)
    dy = torch.randn(B, Lq, N, generator=g).to(torch.bfloat16)
    xg = x.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    y = ops.linear(xg, wg)
    y.backward(dy.to(dev))
    xd = x.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    (xd @ wd.T).backward(dy.double())
    assert_parity(y, (x.double() @ w.double().T), torch.bfloat16, "y")
    assert_parity(xg.grad, xd.grad, torch.bfloat16, "dx")
    assert_parity(wg.grad, wd.grad, torch.bfloat16, "dW")


@pytest.mark.parametrize("bank_dtype,norm", [(torch.bfloat16, None), (torch.bfloat16, "rms")])
def test_kv_weight_grad_per_edge(gpu_device, bank_dtype, norm):
    """Per-edge mode: dkv rows per (sequence, slot) edge, chapters repeated across sequences and one
    skipped edge (out-of-range id) whose rows hold NaN and must not be read."""
    from memory_amd import _lib as L
    from memory_amd import ops
    dev = gpu_device
    T, d, HK, C = 64, 256, 2, 30
    KV2 = 2 * HK * 64
    g = gen(515)
    bank = torch.randn(C * T, d, generator=g)
    chap = torch.randint(0, 12, (3, 5), generator=g).to(torch.int32)  # duplicates across rows
    chap[1, 2] = C + 7                                                 # skipped edge
    E = chap.numel()
    plan = ops.chapter_plan(chap.to(dev), C)
    bg = bank.to(dev, bank_dtype)
    code = ops.norm_code(norm)
    mean = rstd = None
    if code:
        mean, rstd = ops.row_stats(bg, plan, T, code, 1e-5)
    dkv = torch.randn(E * T, KV2, generator=g).to(torch.bfloat16)
    dkv.view(E, T, KV2)[7] = float("nan")  # edge 7 = (1, 2), the skipped one
    dkv_d = dkv.to(dev)
    ws = torch.empty(L.query("moc_kv_wgrad_workspace", KV2, d, E) // 4, device=dev, dtype=torch.float32)
    dw = torch.empty(KV2, d, device=dev, dtype=torch.float32)
    L.call("moc_kv_wgrad", L.ptr(dkv_d), L.ptr(bg), L.dtype_code(bank_dtype), d, T, L.ptr(plan.uniq),
           L.ptr(plan.n_uniq), L.ptr(plan.edge_u), E, L.ptr(mean), L.ptr(rstd), KV2, L.ptr(ws), ws.numel() * 4,
           L.dtype_code(torch.float32), L.ptr(dw), L.stream_ptr(dev))
    ref = torch.zeros(KV2, d, dtype=torch.float64)
    for e, c in enumerate(chap.reshape(-1).tolist()):
        if not 0 <= c < C:
            continue
        X = bg.cpu().double()[c * T:(c + 1) * T]
        if norm == "rms":
            X = O.rms_norm(X, 1e-5)
        ref += dkv.view(E, T, KV2)[e].double().T @ X.to(torch.bfloat16).double()
    assert torch.isfinite(dw).all()
    assert_parity(dw, ref, torch.float32, "dW per edge")


@pytest.mark.parametrize("shape,dtype", [((4097, 768), torch.bfloat16), ((3, 5), torch.bfloat16),
                                         ((1000, 24), torch.float32), ((0, 8), torch.bfloat16)])
def test_zeros_beside(gpu_device, shape, dtype):
    """The side-stream zero fill of the dense bank gradient: every element zero once the
    current stream has waited on the returned event (sizes that are not a multiple of 16
    bytes take the in-order fill)."""
    print(f"zeros_beside {shape} {dtype}", flush=True)
    from memory_amd import ops
    junk = torch.full(shape, 7.0, device=gpu_device, dtype=dtype)
    del junk   # the caching allocator hands the same block out again
    t, ev = ops.zeros_beside(shape, dtype, gpu_device)
    if ev is not None:
        torch.cuda.current_stream(gpu_device).wait_event(ev)
    assert t.shape == shape and t.dtype == dtype
    assert torch.count_nonzero(t).item() == 0


@pytest.mark.parametrize("shape", [(390, 256, 512), (8192, 768, 768)])
def test_rows_linear_matches_fp64(gpu_device, shape):
    """moc_rows_linear (y = x W^T on the chapter GEMM over 64-row blocks) against a float64
    product; rows past R are neither read nor written (the output buffer's tail stays NaN)."""
    from memory_amd import _lib as L
    R, K, N = shape
    g = gen(91)
    x = torch.randn(R, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) / 16).to(torch.bfloat16)
    xd, wd = x.to(gpu_device), w.to(gpu_device)
    y = torch.full((R + 64, N), float("nan"), device=gpu_device, dtype=torch.bfloat16)
    L.call("moc_rows_linear", L.ptr(xd), K, R, L.ptr(wd), N, K, L.ptr(y), N, L.stream_ptr(gpu_device))
    assert_parity(y[:R], x.double() @ w.double().T, torch.bfloat16, "y")
    assert torch.isnan(y[R:].float()).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,Lq,H,HK", [(2, 100, 4, 2), (3, 256, 4, 4), (1, 130, 2, 1)])
def test_dq_with_fused_delta_matches_prep(gpu_device, dtype, B, Lq, H, HK):
    """moc_xattn_bwd_dq_delta (the pre-pass's delta formed inside the dQ kernel) against
    moc_xattn_bwd_prep + moc_xattn_bwd_dq: delta within fp32 rounding of the pre-pass's (the
    summation order differs), padded rows exactly 0, dq within a few units of its last place."""
    print(f"dq_delta dtype={dtype} B={B} L={Lq} H={H} HK={HK}", flush=True)
    from memory_amd import ops, _lib as L
    dev = gpu_device
    g = gen(7 + B + Lq)
    T, S, Dh, C, k, d = 64, 1, 64, 24, 5, 128
    q = torch.randn(B, Lq, H, Dh, generator=g).to(dev, dtype)
    bank = torch.randn(C * T, d, generator=g).to(dev, dtype)
    Wk = (torch.randn(HK * Dh, d, generator=g) / d ** 0.5).to(dev, dtype)
    Wv = (torch.randn(HK * Dh, d, generator=g) / d ** 0.5).to(dev, dtype)
    idx, w, _ = O.route_sequence(torch.randn(B, C, generator=g) * 2, k, S)
    ci, cw = O.prepend_shared_chapters(idx, w, num_chapters=C, num_shared_chapters=S, routed_scaling_factor=2.5)
    out, saved, cfg = ops.routed_attn_forward(q, bank, Wk, Wv, cw.float().to(dev), ci.to(torch.int32).to(dev), C, T,
                                              0, 0.0, HK)
    (qs, _, _, om, outs, lse, kv, _, _, _, _, edge_u, _, _) = saved
    dout = torch.randn(B, Lq, H, Dh, generator=g).to(dev, dtype)
    Lp = lse.shape[2]
    NS = om.shape[1]
    dt = L.dtype_code(dtype)
    st = L.stream_ptr(dev)
    kvl = ops.kv_rows_layout(kv, T, HK, Dh)
    vptr = L.ptr(kv) + HK * Dh * kv.element_size()
    delta_ref = torch.full((B, H, Lp), float("nan"), device=dev)
    L.call("moc_xattn_bwd_prep", dt, L.ptr(qs), L.ptr(outs), L.ptr(dout), B, Lq, H, Dh, L.ptr(delta_ref), None, None, st)
    dq_ref = torch.empty_like(qs)
    L.call("moc_xattn_bwd_dq", dt, L.ptr(qs), L.ptr(kv), vptr, *kvl, L.ptr(edge_u), L.ptr(om), L.ptr(dout),
           L.ptr(lse), L.ptr(delta_ref), B, Lq, H, HK, Dh, T, NS, Dh ** -0.5, L.ptr(dq_ref), st)
    delta = torch.full((B, H, Lp), float("nan"), device=dev)
    dq = torch.empty_like(qs)
    L.call("moc_xattn_bwd_dq_delta", dt, L.ptr(qs), L.ptr(kv), vptr, *kvl, L.ptr(edge_u), L.ptr(om), L.ptr(outs),
           L.ptr(dout), L.ptr(lse), L.ptr(delta), B, Lq, H, HK, Dh, T, NS, Dh ** -0.5, L.ptr(dq), st)
    torch.cuda.synchronize()
    # delta from the rows in double: the fused value and the pre-pass's within fp32 rounding of it
    exact = (dout.double() * outs.double()).sum(-1).permute(0, 2, 1)
    scale = exact.abs().amax().item() + 1e-30
    assert (delta[:, :, :Lq].double() - exact).abs().max().item() <= 1e-5 * scale
    assert (delta_ref[:, :, :Lq].double() - exact).abs().max().item() <= 1e-5 * scale
    assert torch.all(delta[:, :, Lq:] == 0)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    err = (dq.float() - dq_ref.float()).abs().max().item() / (dq_ref.float().abs().max().item() + 1e-30)
    print(f"  delta max |fused - exact| / max|exact| "
          f"{(delta[:, :, :Lq].double() - exact).abs().max().item() / scale:.2e}, dq rel diff {err:.2e}", flush=True)
    assert err <= tol
