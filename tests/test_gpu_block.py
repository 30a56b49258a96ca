"""Caller side of the memory layer on the GPU: the memory_layernorm kernels (RMSNorm of
memory_block.py:18-28 and nn.LayerNorm), the o_proj GEMM with the residual as accumulator
input, and the whole memory sublayer (memory_block.py:549-558) against the oracle in float64.

Tolerances: relative max error fp32 1e-5 / bf16 2e-2, and the parity gate of tests/helpers.py
(fp32 elementwise 1e-4 relative, bf16 max-abs 2e-2)."""

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


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.float32, torch.bfloat16),
                                     (torch.bfloat16, torch.bfloat16)])
@pytest.mark.parametrize("R,d", [(1, 8), (7, 24), (300, 768), (65, 2048), (33, 520)])
def test_row_norm_matches_oracle(dev, norm, xdt, ydt, R, d):
    print(f"row norm {norm} x={xdt} y={ydt} R={R} d={d}", flush=True)
    from memory_amd import ops
    g0 = gen(R * 31 + d)
    x = (torch.randn(R, d, generator=g0) * 2 + 0.5).to(xdt)
    w = torch.randn(d, generator=g0) * 0.5 + 1
    b = torch.randn(d, generator=g0) * 0.1 if norm == "layer" else None
    dy = torch.randn(R, d, generator=g0)
    eps = 1e-5
    xg = x.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    bg = b.to(dev).requires_grad_(True) if b is not None else None
    y = ops.row_norm(xg, wg, bg, eps, norm, ydt)
    assert y.dtype == ydt and y.shape == x.shape
    (y.float() * dy.to(dev)).sum().backward()
    x64 = x.double().requires_grad_(True)
    w64 = w.double().requires_grad_(True)
    b64 = b.double().requires_grad_(True) if b is not None else None
    ref = O.block_rms_norm(x64, w64, eps) if norm == "rms" else F.layer_norm(x64, (d,), w64, b64, eps)
    (ref * dy.double()).sum().backward()
    tol = 1e-5 if (xdt, ydt) == (torch.float32, torch.float32) else 2e-2
    gtol = 1e-5 if xdt == torch.float32 and ydt == torch.float32 else 2e-2
    assert_rel(y.float(), ref.detach(), tol, "y")
    assert_rel(xg.grad.float(), x64.grad, gtol, "dx")
    assert_rel(wg.grad, w64.grad, gtol, "dweight")
    if b is not None:
        assert_rel(bg.grad, b64.grad, gtol, "dbias")
    gate = torch.float32 if (xdt, ydt) == (torch.float32, torch.float32) else torch.bfloat16
    assert_parity(y.float(), ref.detach(), gate, "y")
    assert_parity(xg.grad.float(), x64.grad, gate, "dx")
    assert_parity(wg.grad, w64.grad, gate, "dweight")


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("R,K,N", [(300, 768, 768), (8192, 768, 768), (1000, 512, 256), (129, 256, 768)])
def test_norm_linear_matches_oracle(dev, norm, R, K, N):
    """q_proj(memory_layernorm(x)) as one GEMM (ops.norm_linear: the norm weight folded into the
    projection weight, row statistics inside the GEMM) against float64: output, dx, dweight,
    dbias and dW; rows with a non-zero mean so LayerNorm's centring matters; ragged R."""
    print(f"norm_linear {norm} R={R} K={K} N={N}", flush=True)
    from memory_amd import ops
    g0 = gen(R + K + N)
    x = (torch.randn(R, K, generator=g0) * 2 + 0.5).to(torch.bfloat16)
    w = torch.randn(K, generator=g0) * 0.5 + 1
    b = torch.randn(K, generator=g0) * 0.1 if norm == "layer" else None
    W = (torch.randn(N, K, generator=g0) * K ** -0.5).to(torch.bfloat16)
    dy = torch.randn(R, N, generator=g0)
    eps = 1e-5
    assert ops.norm_linear_supported(x.to(dev), W.to(dev))
    xg, wg, Wg = x.to(dev).requires_grad_(True), w.to(dev).requires_grad_(True), W.to(dev).requires_grad_(True)
    bg = b.to(dev).requires_grad_(True) if b is not None else None
    y = ops.norm_linear(xg, wg, bg, eps, norm, Wg)
    assert y.dtype == torch.bfloat16 and y.shape == (R, N)
    (y.float() * dy.to(dev)).sum().backward()
    x64, w64, W64 = (t.double().requires_grad_(True) for t in (x, w, W))
    b64 = b.double().requires_grad_(True) if b is not None else None
    xn = O.block_rms_norm(x64, w64, eps) if norm == "rms" else F.layer_norm(x64, (K,), w64, b64, eps)
    ref = xn @ W64.t()
    (ref * dy.double()).sum().backward()
    assert_parity(y.float(), ref.detach(), torch.bfloat16, "y")
    assert_parity(xg.grad.float(), x64.grad, torch.bfloat16, "dx")
    assert_parity(wg.grad.float(), w64.grad, torch.bfloat16, "dweight")
    assert_parity(Wg.grad.float(), W64.grad, torch.bfloat16, "dW")
    if b is not None:
        assert_parity(bg.grad.float(), b64.grad, torch.bfloat16, "dbias")


@pytest.mark.parametrize("spread,offset", [(3.0, -1.0), (1.0, 200.0)])
def test_rows_linear_norm_statistics(dev, spread, offset):
    """The row statistics the fused GEMM writes for the norm's backward equal float64's
    (fp32, same eps), for RMSNorm and LayerNorm; the second case has rows whose mean is 200 times
    their spread, where a variance taken as E[x^2] - mean^2 in fp32 loses ~15 bits."""
    from memory_amd import _lib as L
    g0 = gen(3)
    R, K, N = 333, 768, 256
    x = (torch.randn(R, K, generator=g0) * spread + offset).to(torch.bfloat16).to(dev)
    W = (torch.randn(N, K, generator=g0) * 0.05).to(torch.bfloat16).to(dev)
    gamma = torch.ones(K, device=dev)
    beta = torch.zeros(K, device=dev)
    st = L.stream_ptr(dev)
    for norm in (L.MOC_NORM_RMS, L.MOC_NORM_LAYERNORM):
        ln = norm == L.MOC_NORM_LAYERNORM
        wf = torch.empty_like(W)
        u = torch.empty(N, device=dev) if ln else None
        v = torch.empty(N, device=dev) if ln else None
        L.call("moc_norm_fold_weight", L.ptr(W), N, K, L.ptr(gamma), L.ptr(beta if ln else None), L.ptr(wf),
               L.ptr(u), L.ptr(v), st)
        assert torch.equal(wf, W)   # unit gamma: the folded weight is the weight
        y = torch.empty(R, N, device=dev, dtype=torch.bfloat16)
        mean, rstd = torch.empty(R, device=dev), torch.empty(R, device=dev)
        L.call("moc_rows_linear_norm", L.ptr(x), K, R, L.ptr(wf), N, K, norm, 1e-5, L.ptr(u), L.ptr(v), L.ptr(y), N,
               L.ptr(mean), L.ptr(rstd), st)
        x64 = x.double()
        m64 = x64.mean(-1) if ln else torch.zeros(R, dtype=torch.float64, device=dev)
        var = ((x64 - m64[:, None]) ** 2).mean(-1) if ln else (x64 ** 2).mean(-1)
        assert_rel(rstd.double(), 1 / torch.sqrt(var + 1e-5), 1e-5, "rstd")
        if ln:
            assert_rel(mean.double(), m64, 1e-5, "mean")


@pytest.mark.parametrize("rdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(3, 40, 64), (2, 520, 768)])
def test_linear_residual(dev, rdt, shape):
    """residual + o_proj(x) (memory_block.py:549-558); at d = 768 in bf16 the residual rides in
    the chapter GEMM's epilogue (moc_rows_linear_residual) and dx runs on the rows GEMM."""
    from memory_amd import ops
    g0 = gen(5)
    B, T, d = shape
    x = torch.randn(B, T, d, generator=g0).to(torch.bfloat16)
    W = (torch.randn(d, d, generator=g0) * d ** -0.5).to(torch.bfloat16)
    r = torch.randn(B, T, d, generator=g0).to(rdt)
    dy = torch.randn(B, T, d, generator=g0)
    xg, Wg, rg = (t.to(dev).requires_grad_(True) for t in (x, W, r))
    out = ops.linear_residual(xg, Wg, rg)
    assert out.dtype == rdt
    (out.float() * dy.to(dev)).sum().backward()
    x64, W64, r64 = (t.double().requires_grad_(True) for t in (x, W, r))
    ref = r64 + x64 @ W64.t()
    (ref * dy.double()).sum().backward()
    assert_parity(out.float(), ref.detach(), torch.bfloat16, "out")   # bf16 product (+ residual)
    assert_parity(xg.grad.float(), x64.grad, torch.bfloat16, "dx")
    assert_parity(Wg.grad.float(), W64.grad, torch.bfloat16, "dW")
    assert_rel(rg.grad.float(), r64.grad, 1e-6 if rdt == torch.float32 else 1e-2, "dresidual")


@pytest.mark.parametrize("dtype,use_rms,d", [(torch.float32, True, 128), (torch.float32, False, 128),
                                             (torch.bfloat16, True, 128), (torch.bfloat16, False, 128),
                                             (torch.bfloat16, True, 256), (torch.bfloat16, False, 256)])
def test_memory_sublayer_matches_oracle(dev, dtype, use_rms, d):
    """residual + memory_attn(memory_layernorm(h)) over routed chapters of a bank (the fused
    routed_memory_state path): output and every gradient (h, norm weight / bias, q/k/v/o
    weights, bank) against the oracle's sublayer on the gathered, omega-weighted memory.  At
    d = 256 in bf16 the norm runs inside the q projection's GEMM (ops.norm_linear)."""
    print(f"memory sublayer {dtype} rms={use_rms} d={d}", flush=True)
    from memory_amd import ops
    from memory_amd.memory_block import MemorySublayer
    B, L, H, C, T, k, S = 2, 70, d // 64, 9, 64, 3, 1
    g0 = gen(77 + int(use_rms))
    h = torch.randn(B, L, d, generator=g0).to(dtype)
    bank = (torch.randn(C * T, d, generator=g0) * 0.5).to(dtype)
    nw = torch.randn(d, generator=g0) * 0.2 + 1
    nb = torch.randn(d, generator=g0) * 0.1
    Wq, Wk, Wv, Wo = ((torch.randn(d, d, generator=g0) * d ** -0.5).to(dtype) for _ in range(4))
    dO = torch.randn(B, L, d, generator=g0)
    logits = torch.randn(B, C, generator=g0)
    idx, w, _ = O.route_sequence(logits, k, S)
    ci, cw = O.prepend_shared_chapters(idx, w, num_chapters=C, num_shared_chapters=S, routed_scaling_factor=2.5)

    sub = MemorySublayer(d, H, use_rms_norm=use_rms, norm_eps=1e-5, wo_init_zero=False)
    with torch.no_grad():
        sub.memory_layernorm.weight.copy_(nw)
        if not use_rms:
            sub.memory_layernorm.bias.copy_(nb)
        for lin, W in ((sub.memory_attn.q_proj, Wq), (sub.memory_attn.k_proj, Wk), (sub.memory_attn.v_proj, Wv),
                       (sub.memory_attn.o_proj, Wo)):
            lin.weight.copy_(W.float())
    sub = sub.to(dev)
    for lin in (sub.memory_attn.q_proj, sub.memory_attn.k_proj, sub.memory_attn.v_proj, sub.memory_attn.o_proj):
        lin.to(dtype)
    hg = h.to(dev).requires_grad_(True)
    bg = bank.to(dev).requires_grad_(True)
    assert ops.norm_linear_supported(hg, sub.memory_attn.q_proj.weight) == (dtype == torch.bfloat16 and d == 256)
    state = {"bank": bg, "chapter_indices": ci.to(dev), "chapter_weights": cw.to(dev), "num_chapters": C,
             "tokens_per_chapter": T}
    out = sub(hg, routed_memory_state=state)
    assert out.dtype == dtype
    (out.float() * dO.to(dev)).sum().backward()

    leaves = [t.double().requires_grad_(True) for t in (h, bank, nw, nb, Wq, Wk, Wv, Wo)]
    h64, bank64, nw64, nb64, Wq64, Wk64, Wv64, Wo64 = leaves
    mem, _ = O.gather_chapters(bank64, ci, T)
    mem = O.weight_memory(mem, cw.double(), T)
    ref = O.memory_sublayer(h64, nw64, None if use_rms else nb64, 1e-5, use_rms, mem, Wq64, Wk64, Wv64, Wo64, H, H)
    (ref * dO.double()).sum().backward()
    assert_parity(out.float(), ref.detach(), dtype, "out")
    names = ["dh", "dbank", "dnorm_w", "dnorm_b", "dWq", "dWk", "dWv", "dWo"]
    got = [hg.grad, bg.grad, sub.memory_layernorm.weight.grad,
           None if use_rms else sub.memory_layernorm.bias.grad, sub.memory_attn.q_proj.weight.grad,
           sub.memory_attn.k_proj.weight.grad, sub.memory_attn.v_proj.weight.grad, sub.memory_attn.o_proj.weight.grad]
    for n, gr, r in zip(names, got, leaves):
        if gr is None:
            continue
        assert_parity(gr.float(), r.grad, dtype, n)
