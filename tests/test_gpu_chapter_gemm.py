"""Chapter GEMMs of the K/V path (moc_chapter_project, moc_chapter_dx, moc_weight_pack) against
float64 references of the reference's math: the gather + k_proj/v_proj of
memory_transformer/memory_bank.py:263-293 and memory_attention.py:241-243, and its input gradient
scattered into the bank (memory_bank.py:287-291)."""

import pytest
import torch

from helpers import assert_parity, gen

pytestmark = pytest.mark.gpu


def _ops():
    from memory_amd import ops
    return ops


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    return torch.device("cuda", 0)


@pytest.mark.parametrize("wdt", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
                                 (torch.float32, torch.bfloat16)])
def test_weight_pack_exact(dev, wdt):
    ops = _ops()
    wk = torch.randn(192, 320, generator=gen(1)).to(wdt[0])
    wv = torch.randn(192, 320, generator=gen(2)).to(wdt[1])
    wkv, wkv_t = ops.weight_pack(wk.to(dev), wv.to(dev), rows=True, transposed=True)
    ref = torch.cat([wk.to(torch.bfloat16), wv.to(torch.bfloat16)])
    assert torch.equal(wkv.cpu(), ref)
    assert torch.equal(wkv_t.cpu(), ref.t().contiguous())
    _, only_t = ops.weight_pack(wk.to(dev), wv.to(dev), rows=False, transposed=True)
    assert torch.equal(only_t.cpu(), ref.t().contiguous())


@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("N,K,ldt", [(4097, 768, 4352), (200, 64, 200), (37, 136, 48)])
def test_weight_transpose_exact(dev, wdt, N, K, ldt):
    """moc_weight_transpose: wt [K][ldt] = bf16(w)^T with zero columns N .. ldt-1, bit for bit
    (the per-token router's padded W^T)."""
    from memory_amd import _lib as L
    from memory_amd._lib import call, ptr, stream_ptr
    w = torch.randn(N, K, generator=gen(N + K)).to(wdt)
    wd = w.to(dev)
    wt = torch.full((K, ldt), 7.0, device=dev, dtype=torch.bfloat16)
    call("moc_weight_transpose", ptr(wd), L.dtype_code(wdt), N, K, ptr(wt), ldt, stream_ptr(dev))
    ref = torch.zeros(K, ldt, dtype=torch.bfloat16)
    ref[:, :N] = w.to(torch.bfloat16).t()
    assert torch.equal(wt.cpu(), ref)


def _plan(ops, dev, chap, C):
    return ops.chapter_plan(torch.as_tensor(chap, dtype=torch.int32).to(dev), C)


# (C, d, N, chap) -- N = 2*HK*Dh; the second case spans many tiles, every XCD range, a
# row block with fewer than 4 chapters and unused plan slots
_PROJ_CASES = [
    (40, 256, 256, [[0, 7, 3, 39], [0, 3, 11, 25], [0, 39, 38, 1]]),
    (700, 768, 1536, "random"),
]


@pytest.mark.parametrize("case", range(len(_PROJ_CASES)))
@pytest.mark.parametrize("gather", [True, False])
def test_chapter_project(dev, case, gather):
    ops = _ops()
    C, d, N, chap = _PROJ_CASES[case]
    T = 64
    if chap == "random":
        g = gen(5)
        chap = torch.cat([torch.zeros(8, 1, dtype=torch.int64),
                          torch.stack([torch.randperm(C - 1, generator=g)[:40] + 1 for _ in range(8)])], 1)
    bank = (torch.randn(C * T, d, generator=gen(6)) * 0.5).to(torch.bfloat16)
    w = (torch.randn(N, d, generator=gen(7)) / d ** 0.5).to(torch.bfloat16)
    plan = _plan(ops, dev, chap, C)
    n_u = int(plan.n_uniq[0])
    uniq = plan.uniq[:n_u].cpu().long()
    X = bank.view(C, T, d)[uniq].reshape(-1, d)
    bg = bank.to(dev)
    if gather:
        rows = bg
    else:
        rows = torch.zeros(plan.max_u * T, d, dtype=torch.bfloat16)
        rows[: n_u * T] = X
        rows = rows.to(dev)
    y = ops.chapter_project(rows, plan, w.to(dev), gather=gather)
    ref = X.double() @ w.double().t()
    print(f"C={C} d={d} N={N} n_uniq={n_u} max_u={plan.max_u} gather={gather}")
    assert_parity(y[: n_u * T].cpu(), ref, torch.bfloat16, "projection rows")
    # bf16 rounding of fp32 sums: no element further than one bf16 ulp of the result
    err = (y[: n_u * T].cpu().double() - ref).abs()
    assert (err <= ref.abs() * 2 ** -8 + 1e-3).all(), err.max().item()


def _dx_case(C, NSEQ, NS, seed):
    g = gen(seed)
    rows = [torch.cat([torch.zeros(1, dtype=torch.int64), torch.randint(1, C, (NS - 1,), generator=g)])
            for _ in range(NSEQ)]
    return torch.stack(rows)   # chapter 0 in every sequence, random collisions elsewhere


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bank_rows", [True, False])
@pytest.mark.parametrize("shape", [(60, 4, 9, 256, 512), (600, 8, 65, 768, 1536)])
def test_chapter_dx(dev, out_dtype, bank_rows, shape):
    ops = _ops()
    C, NSEQ, NS, d, K = shape
    T = 64
    chap = _dx_case(C, NSEQ, NS, 11)
    E = chap.numel()
    plan = _plan(ops, dev, chap, C)
    n_u = int(plan.n_uniq[0])
    uniq = plan.uniq[:n_u].cpu().long()
    dkv = torch.randn(E * T, K, generator=gen(12)).to(torch.bfloat16)
    wkv = (torch.randn(K, d, generator=gen(13)) / K ** 0.5).to(torch.bfloat16)
    _, wkv_t = ops.weight_pack(wkv[: K // 2].to(dev), wkv[K // 2:].to(dev), rows=False, transposed=True)
    flat = chap.reshape(-1)
    ref_c = torch.zeros(n_u, T, d, dtype=torch.float64)
    for u in range(n_u):
        edges = (flat == uniq[u]).nonzero().view(-1)
        s = sum(dkv[e * T:(e + 1) * T].double() for e in edges.tolist())
        ref_c[u] = s @ wkv.double()
    counts = torch.bincount(flat, minlength=C)
    assert counts.max() > 1 and (counts == 1).any()   # both code paths (summed and in-place)
    if bank_rows:
        out = torch.zeros(C * T, d, device=dev, dtype=out_dtype)
    else:
        out = torch.full((plan.max_u * T, d), float("nan"), device=dev, dtype=out_dtype)
    dkv_d = dkv.to(dev)
    red = ops.dkv_multi_reduce(dkv_d, plan.n_uniq, plan.max_u, plan.csr_off, plan.csr_edge)
    ops.chapter_dx(dkv_d, red, plan.uniq, plan.n_uniq, plan.max_u, plan.csr_off, plan.csr_edge, wkv_t, out,
                   bank_rows=bank_rows)
    o = out.cpu()
    print(f"C={C} E={E} n_uniq={n_u} d={d} K={K} out={out_dtype} bank_rows={bank_rows}")
    if bank_rows:
        got = o.view(C, T, d)[uniq]
        mask = torch.ones(C, dtype=torch.bool)
        mask[uniq] = False
        assert (o.view(C, T, d)[mask] == 0).all(), "rows of unselected chapters must stay zero"
    else:
        got = o[: n_u * T].view(n_u, T, d)
        if plan.max_u > n_u:
            assert torch.isnan(o[n_u * T:].float()).all(), "unused plan slots must not be written"
    assert_parity(got, ref_c, torch.bfloat16, "dX per chapter")


@pytest.mark.parametrize("gather", [True, False])
@pytest.mark.parametrize("shape", [(60, 4, 9, 256, 512), (600, 8, 65, 768, 1536)])
def test_chapter_wgrad(dev, gather, shape):
    """dW = sum over distinct chapters of (sum of the chapter's edge rows)^T X_c: the weight
    gradient of k_proj / v_proj over the gathered rows (memory_attention.py:241-243)."""
    ops = _ops()
    from memory_amd import _lib as L
    C, NSEQ, NS, d, K = shape
    T = 64
    chap = _dx_case(C, NSEQ, NS, 21)
    E = chap.numel()
    plan = _plan(ops, dev, chap, C)
    n_u = int(plan.n_uniq[0])
    uniq = plan.uniq[:n_u].cpu().long()
    dkv = torch.randn(E * T, K, generator=gen(22)).to(torch.bfloat16)
    bank = torch.randn(C * T, d, generator=gen(23)).to(torch.bfloat16)
    flat = chap.reshape(-1)
    ref = torch.zeros(K, d, dtype=torch.float64)
    for u in range(n_u):
        edges = (flat == uniq[u]).nonzero().view(-1)
        s = sum(dkv[e * T:(e + 1) * T].double() for e in edges.tolist())
        ref += s.t() @ bank.view(C, T, d)[uniq[u]].double()
    dkv_d = dkv.to(dev)
    red = ops.dkv_multi_reduce(dkv_d, plan.n_uniq, plan.max_u, plan.csr_off, plan.csr_edge)
    if gather:
        xs = bank.to(dev)
    else:
        xs = torch.zeros(plan.max_u * T, d, dtype=torch.bfloat16)
        xs[: n_u * T] = bank.view(C, T, d)[uniq].reshape(-1, d)
        xs = xs.to(dev)
    ws_bytes = L.query("moc_chapter_wgrad_workspace", K, d, plan.max_u)
    ws = torch.empty(ws_bytes // 4, device=dev)
    for out_dtype in (torch.float32, torch.bfloat16):
        dw = torch.empty(K, d, device=dev, dtype=out_dtype)
        L.call("moc_chapter_wgrad", dkv_d.data_ptr(), K, red.data_ptr(), xs.data_ptr(), xs.stride(0), int(gather),
               plan.uniq.data_ptr(), plan.n_uniq.data_ptr(), plan.max_u, plan.csr_off.data_ptr(),
               plan.csr_edge.data_ptr(), K, d, ws.data_ptr(), ws_bytes, L.dtype_code(out_dtype), dw.data_ptr(),
               torch.cuda.current_stream().cuda_stream)
        print(f"C={C} E={E} n_uniq={n_u} d={d} K={K} gather={gather} out={out_dtype}")
        assert_parity(dw.cpu(), ref, torch.bfloat16, "dW")


@pytest.mark.parametrize("shape", [(8192, 768, 768), (1000, 512, 256), (980, 256, 512)])
def test_dense_wgrad_lds_dma_path(dev, shape):
    """moc_linear_wgrad on bf16 operands with N, K multiples of 256 (the chapter weight-gradient
    kernel, rows past R reading zero) against a float64 product."""
    ops = _ops()
    R, N, K = shape
    dy = torch.randn(R, N, generator=gen(31)).to(torch.bfloat16)
    x = torch.randn(R, K, generator=gen(32)).to(torch.bfloat16)
    dw = ops.linear_wgrad(dy.to(dev), x.to(dev), torch.float32)
    ref = dy.double().t() @ x.double()
    print(f"R={R} N={N} K={K}")
    assert_parity(dw.cpu(), ref, torch.bfloat16, "dW dense")


# rows GEMM (moc_rows_linear): (R, N, K) -- the first two take the wide 256-row tiles (>= 2 rounds
# of the persistent grid: the token path's K/V projection and its dX at reduced R, ragged last
# block), the third the 128-row tiles
@pytest.mark.parametrize("shape", [(70000, 1536, 768), (65600, 768, 1536), (1000, 768, 768)])
def test_rows_linear(dev, shape):
    """y = x W^T over contiguous rows (the token path's whole-bank K/V projection and its input
    gradient, memory_attention.py:241-243) against a float64 product; rows past R untouched."""
    ops = _ops()
    R, N, K = shape
    x = torch.randn(R, K, generator=gen(41)).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=gen(42)) / K ** 0.5).to(torch.bfloat16)
    out = torch.full((R + 64, N), float("nan"), device=dev, dtype=torch.bfloat16)
    ops.rows_linear(x.to(dev), w.to(dev), out=out[:R])
    ref = x.double() @ w.double().t()
    got = out[:R].cpu()
    print(f"R={R} N={N} K={K}")
    assert_parity(got, ref, torch.bfloat16, "rows linear")
    err = (got.double() - ref).abs()
    assert (err <= ref.abs() * 2 ** -8 + 1e-3).all(), err.max().item()
    assert torch.isnan(out[R:].float().cpu()).all(), "rows past R must not be written"


@pytest.mark.parametrize("shape", [(8192, 768, 768), (1000, 256, 512), (40000, 768, 768)])
def test_rows_linear_residual(dev, shape):
    """out = residual + x W^T in one GEMM (memory_block.py:549-558 with the o_proj of
    memory_attention.py:456): one rounding of the fp32 sum, checked against float64; also in
    place (residual buffer = output)."""
    from memory_amd import _lib as L
    R, N, K = shape
    x = torch.randn(R, K, generator=gen(51)).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=gen(52)) / K ** 0.5).to(torch.bfloat16)
    res = (torch.randn(R, N, generator=gen(53)) * 4).to(torch.bfloat16)
    ref = res.double() + x.double() @ w.double().t()
    xd, wd, rd = x.to(dev), w.to(dev), res.to(dev)
    st = torch.cuda.current_stream().cuda_stream
    y = torch.empty(R, N, device=dev, dtype=torch.bfloat16)
    L.call("moc_rows_linear_residual", xd.data_ptr(), K, R, wd.data_ptr(), N, K, rd.data_ptr(), N, y.data_ptr(), N, st)
    print(f"R={R} N={N} K={K}")
    assert_parity(y.cpu(), ref, torch.bfloat16, "rows linear + residual")
    err = (y.cpu().double() - ref).abs()
    assert (err <= ref.abs() * 2 ** -8 + 1e-3).all(), err.max().item()
    L.call("moc_rows_linear_residual", xd.data_ptr(), K, R, wd.data_ptr(), N, K, rd.data_ptr(), N, rd.data_ptr(), N,
           st)
    assert torch.equal(rd.cpu(), y.cpu()), "in place must equal out of place"


@pytest.mark.parametrize("shape", [(8192, 4097, 768), (300, 4097, 768), (700, 100, 128), (8192, 4096, 768)])
@pytest.mark.parametrize("bias", [True, False])
def test_rows_linear_f32_any_n(dev, shape, bias):
    """fp32 logits x W^T + b for any number of chapters (router.py:294 ``self.router(h)`` with bf16
    operands): columns past N and rows past R untouched, within fp32 rounding of float64."""
    from memory_amd import _lib as L
    R, N, K = shape
    x = torch.randn(R, K, generator=gen(61)).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=gen(62)) * 0.02).to(torch.bfloat16)
    b = torch.randn(N, generator=gen(63))
    ldy = N + 3
    y = torch.full((R + 1, ldy), float("nan"), device=dev)
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    L.call("moc_rows_linear_f32", xd.data_ptr(), K, R, wd.data_ptr(), N, K,
           bd.data_ptr() if bias else None, y.data_ptr(), ldy, torch.cuda.current_stream().cuda_stream)
    ref = x.double() @ w.double().t() + (b.double() if bias else 0.0)
    yc = y.cpu()
    print(f"R={R} N={N} K={K} bias={bias}")
    assert_parity(yc[:R, :N], ref, torch.float32, "logits")
    assert torch.isnan(yc[:R, N:]).all() and torch.isnan(yc[R:]).all(), "outside [R, N] must stay untouched"
