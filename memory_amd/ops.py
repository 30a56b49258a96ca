"""Autograd functions over the libmoc kernels.

Every function here runs HIP kernels through the C ABI (memory_amd/_lib.py);
tensors must live on a ROCm device.  PyTorch provides device memory (caching
allocator), the current stream and autograd bookkeeping only.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F

from . import _lib as L
from ._lib import call, ptr, stream_ptr


# --------------------------------------------------------------------------- router

class _RouterPool(torch.autograd.Function):
    """Mean (or coefficient-weighted) pooling over the sequence, fp32 output.

    Reference: memory_transformer/router.py:96-107 (mean) and :158-195 (rolling
    mean, which is a fixed linear combination of positions)."""

    @staticmethod
    def forward(ctx, h: torch.Tensor, coef: Optional[torch.Tensor]):
        L.require_gpu(h)
        h = h.contiguous()
        B, Lq, d = h.shape
        pooled = torch.empty(B, d, device=h.device, dtype=torch.float32)
        ws_bytes = L.query("moc_router_pool_workspace", B, Lq, d)
        ws = torch.empty(max(1, ws_bytes), device=h.device, dtype=torch.uint8)
        cf = None if coef is None else coef.to(device=h.device, dtype=torch.float32).contiguous()
        call("moc_router_pool", ptr(h), L.dtype_code(h.dtype), B, Lq, d, ptr(cf), ptr(pooled), ptr(ws), ws_bytes,
             stream_ptr(h.device))
        ctx.save_for_backward(cf)
        ctx.shape, ctx.dtype = (B, Lq, d), h.dtype
        return pooled

    @staticmethod
    def backward(ctx, dpooled):
        (cf,) = ctx.saved_tensors
        B, Lq, d = ctx.shape
        if cf is None:
            dh = (dpooled * (1.0 / Lq)).to(ctx.dtype).unsqueeze(1).expand(B, Lq, d)
        else:
            dh = (dpooled.unsqueeze(1) * cf.view(1, Lq, 1)).to(ctx.dtype)
        return dh, None


def router_pool(h: torch.Tensor, coef: Optional[torch.Tensor] = None) -> torch.Tensor:
    return _RouterPool.apply(h, coef)


class _RouterLinear(torch.autograd.Function):
    """logits = x W^T + b in fp32 for a few rows (sequence-level routing)."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, W: torch.Tensor, b: Optional[torch.Tensor]):
        L.require_gpu(x, W, b)
        x = x.float().contiguous()
        Wc = W.contiguous()
        bc = None if b is None else b.float().contiguous()
        R, d = x.shape
        C = W.shape[0]
        logits = torch.empty(R, C, device=x.device, dtype=torch.float32)
        call("moc_router_linear", ptr(x), R, d, ptr(Wc), L.dtype_code(Wc.dtype), ptr(bc), C, ptr(logits),
             stream_ptr(x.device))
        ctx.save_for_backward(x, Wc)
        ctx.has_b = b is not None
        ctx.b_dtype = None if b is None else b.dtype
        return logits

    @staticmethod
    def backward(ctx, dz):
        x, Wc = ctx.saved_tensors
        dz = dz.float().contiguous()
        R, d = x.shape
        C = Wc.shape[0]
        need_x, need_w, need_b = ctx.needs_input_grad
        dx = torch.empty(R, d, device=x.device, dtype=torch.float32) if need_x else None
        dW = torch.empty(C, d, device=x.device, dtype=torch.float32) if need_w else None
        db = torch.empty(C, device=x.device, dtype=torch.float32) if (need_b and ctx.has_b) else None
        ws = None
        if dx is not None:
            ws = torch.empty(L.query("moc_router_linear_bwd_workspace", R, d, C) // 4, device=x.device,
                             dtype=torch.float32)
        # one pass over W: dW, db and dx (partials over chapter blocks, summed in order)
        call("moc_router_linear_bwd", ptr(dz), ptr(x), R, d, ptr(Wc), L.dtype_code(Wc.dtype), C, ptr(dx), ptr(dW),
             ptr(db), ptr(ws), 0 if ws is None else ws.numel() * 4, stream_ptr(x.device))
        if dW is not None:
            dW = dW.to(Wc.dtype)
        if db is not None:
            db = db.to(ctx.b_dtype)
        return dx, dW, db


def router_linear(x: torch.Tensor, W: torch.Tensor, b: Optional[torch.Tensor]) -> torch.Tensor:
    return _RouterLinear.apply(x, W, b)


class _RouterTopK(torch.autograd.Function):
    """softmax -> shared-prefix mask -> renorm -> top-k -> renorm (router.py:114-149)."""

    @staticmethod
    def forward(ctx, logits: torch.Tensor, k: int, S: int):
        L.require_gpu(logits)
        logits = logits.float().contiguous()
        R, C = logits.shape
        idx = torch.empty(R, k, device=logits.device, dtype=torch.int32)
        w = torch.empty(R, k, device=logits.device, dtype=torch.float32)
        call("moc_router_topk", ptr(logits), R, C, S, k, ptr(idx), ptr(w), None, stream_ptr(logits.device))
        ctx.save_for_backward(logits, idx)
        ctx.k, ctx.S = k, S
        ctx.mark_non_differentiable(idx)
        ctx.set_materialize_grads(False)   # no zero-filled gradient for the int ids
        return idx, w

    @staticmethod
    def backward(ctx, _didx, dw):
        logits, idx = ctx.saved_tensors
        R, C = logits.shape
        dz = torch.empty_like(logits)
        if dw is None:
            return None, None, None
        dw = dw.float().contiguous()
        call("moc_router_topk_bwd", ptr(logits), ptr(idx), ptr(dw), R, C, ctx.S, ctx.k, ptr(dz),
             stream_ptr(logits.device))
        return dz, None, None


def router_topk(logits: torch.Tensor, k: int, exclude_prefix_chapters: int = 0):
    """Returns (idx int32 (R, k) global chapter ids, weights fp32 (R, k))."""
    return _RouterTopK.apply(logits, int(k), int(exclude_prefix_chapters))


class _PrependShared(torch.autograd.Function):
    """MemoryTransformer._prepend_shared_chapters (memory_transformer/model.py:356-391)."""

    @staticmethod
    def forward(ctx, idx: torch.Tensor, w: torch.Tensor, S: int, scale: float):
        L.require_gpu(idx, w)
        idx = idx.to(torch.int32).contiguous()
        w = w.float().contiguous()
        R, k = idx.shape
        idx_star = torch.empty(R, S + k, device=idx.device, dtype=torch.int32)
        omega = torch.empty(R, S + k, device=idx.device, dtype=torch.float32)
        call("moc_prepend_shared", ptr(idx), ptr(w), R, k, S, float(scale), ptr(idx_star), ptr(omega),
             stream_ptr(idx.device))
        ctx.save_for_backward(w)
        ctx.S, ctx.scale = S, float(scale)
        ctx.mark_non_differentiable(idx_star)
        ctx.set_materialize_grads(False)   # no zero-filled gradient for the int ids
        return idx_star, omega

    @staticmethod
    def backward(ctx, _di, domega):
        (w,) = ctx.saved_tensors
        R, k = w.shape
        if domega is None or k == 0:
            return None, None, None, None
        dw = torch.empty_like(w)
        dom = domega.float().contiguous()  # held until the launch is enqueued
        call("moc_prepend_shared_bwd", ptr(w), ptr(dom), R, k, ctx.S, ctx.scale, ptr(dw), stream_ptr(w.device))
        return None, dw, None, None


def prepend_shared(idx: torch.Tensor, w: torch.Tensor, num_shared: int, routed_scale: float):
    return _PrependShared.apply(idx, w, int(num_shared), float(routed_scale))


# ----------------------------------------------------------------------- chapter plan

@dataclass
class ChapterPlan:
    uniq: torch.Tensor      # int32 [max_u]
    n_uniq: torch.Tensor    # int32 [2]  (distinct chapters, skipped edges)
    edge_u: torch.Tensor    # int32 [E]
    csr_off: torch.Tensor   # int32 [max_u + 1]
    csr_edge: torch.Tensor  # int32 [E]
    max_u: int
    num_chapters: int


def chapter_plan(chap: torch.Tensor, num_chapters: int) -> ChapterPlan:
    """De-duplicate the selected chapters (any shape, flattened row-major into edges)."""
    L.require_gpu(chap)
    flat = chap.reshape(-1).to(torch.int32).contiguous()
    E = flat.numel()
    C = int(num_chapters)
    max_u = min(E, C)
    dev = flat.device
    uniq = torch.empty(max_u, device=dev, dtype=torch.int32)
    n_uniq = torch.empty(2, device=dev, dtype=torch.int32)
    edge_u = torch.empty(E, device=dev, dtype=torch.int32)
    csr_off = torch.empty(max_u + 1, device=dev, dtype=torch.int32)
    csr_edge = torch.empty(E, device=dev, dtype=torch.int32)
    ws_bytes = L.query("moc_chapter_plan_workspace", E, C)
    ws = torch.empty(max(1, ws_bytes), device=dev, dtype=torch.uint8)
    call("moc_chapter_plan", ptr(flat), E, C, ptr(ws), ws_bytes, ptr(uniq), ptr(n_uniq), ptr(edge_u), ptr(csr_off),
         ptr(csr_edge), stream_ptr(dev))
    return ChapterPlan(uniq, n_uniq, edge_u, csr_off, csr_edge, max_u, C)


def identity_plan(num_chapters: int, device) -> ChapterPlan:
    """The plan of edges 0 .. C-1 selecting chapters 0 .. C-1 (every chapter once, in order),
    written directly: what moc_chapter_plan returns for arange(C)."""
    C = int(num_chapters)
    ar = torch.arange(C + 1, device=device, dtype=torch.int32)
    n_uniq = torch.full((2,), C, device=device, dtype=torch.int32)   # {C, 0} without a host copy
    n_uniq[1:].zero_()
    return ChapterPlan(ar[:C], n_uniq, ar[:C], ar, ar[:C], C, C)


_NORM = {None: L.MOC_NORM_NONE, "none": L.MOC_NORM_NONE, "rms": L.MOC_NORM_RMS, "layernorm": L.MOC_NORM_LAYERNORM}


def norm_code(norm_type: Optional[str]) -> int:
    if norm_type not in _NORM:
        raise ValueError(f"Unsupported norm_type: {norm_type}")
    return _NORM[norm_type]


def row_stats(bank: torch.Tensor, plan: ChapterPlan, T: int, norm: int, eps: float):
    rows = plan.max_u * T
    mean = torch.empty(rows, device=bank.device, dtype=torch.float32)
    rstd = torch.empty(rows, device=bank.device, dtype=torch.float32)
    call("moc_row_stats", ptr(bank), L.dtype_code(bank.dtype), bank.shape[1], T, ptr(plan.uniq), ptr(plan.n_uniq),
         plan.max_u, norm, float(eps), ptr(mean), ptr(rstd), stream_ptr(bank.device))
    return mean, rstd


def kv_project(bank: torch.Tensor, plan: ChapterPlan, T: int, wkv: torch.Tensor, HK: int, Dh: int,
               mean: Optional[torch.Tensor], rstd: Optional[torch.Tensor], dtype: torch.dtype,
               layouts=("k", "v")):
    """Chapter-head tiles of the plan's chapters.  ``layouts`` picks the outputs among
    "k", "v" ([u][hk][t][dh]) and "kt", "vt" (transposed, [u][hk][dh][t])."""
    out = {}
    for name in ("k", "v", "kt", "vt"):
        if name in layouts:
            out[name] = torch.empty(plan.max_u, HK, T, Dh, device=bank.device, dtype=dtype)
    call("moc_kv_project", L.dtype_code(dtype), ptr(bank), L.dtype_code(bank.dtype), bank.shape[1], T, ptr(plan.uniq),
         ptr(plan.n_uniq), plan.max_u, ptr(mean), ptr(rstd), ptr(wkv), HK, Dh, ptr(out.get("k")), ptr(out.get("v")),
         ptr(out.get("kt")), ptr(out.get("vt")), stream_ptr(bank.device))
    return tuple(out[n] for n in layouts)


def weight_pack(wk: torch.Tensor, wv: torch.Tensor, rows: bool = True, transposed: bool = False):
    """[Wk; Wv] in bf16 ([2*KV][d]) and / or its transpose ([d][2*KV]) in one kernel (the
    concatenated K/V weight of the chapter GEMMs).  Returns (wkv or None, wkv_t or None)."""
    wk = wk.contiguous()
    wv = wv.contiguous()
    KV, d = wk.shape
    dev = wk.device
    wkv = torch.empty(2 * KV, d, device=dev, dtype=torch.bfloat16) if rows else None
    wkv_t = torch.empty(d, 2 * KV, device=dev, dtype=torch.bfloat16) if transposed else None
    call("moc_weight_pack", ptr(wk), L.dtype_code(wk.dtype), ptr(wv), L.dtype_code(wv.dtype), KV, d, ptr(wkv),
         ptr(wkv_t), stream_ptr(dev))
    return wkv, wkv_t


def chapter_project(rows: torch.Tensor, plan: ChapterPlan, wkv: torch.Tensor, gather: bool) -> torch.Tensor:
    """Projection rows [max_u * 64][2*KV] (bf16) of the plan's distinct chapters: rows are the
    bank (gather) or a contiguous [max_u * 64][d] block; wkv [2*KV][d] bf16."""
    N, K = wkv.shape
    y = torch.empty(plan.max_u * 64, N, device=rows.device, dtype=torch.bfloat16)
    call("moc_chapter_project", ptr(rows), rows.stride(0), 1 if gather else 0, ptr(plan.uniq), ptr(plan.n_uniq),
         plan.max_u, ptr(wkv), N, K, ptr(y), N, stream_ptr(rows.device))
    return y


def dkv_multi_reduce(dkv_edge: torch.Tensor, n_uniq, max_u: int, csr_off, csr_edge) -> torch.Tensor:
    """Sums of the dK|dV rows of the chapters selected by several edges ([max_u * 64][2*KV]
    bf16; rows of single-edge chapters are not written)."""
    K = dkv_edge.shape[1]
    red = torch.empty(max_u * 64, K, device=dkv_edge.device, dtype=torch.bfloat16)
    call("moc_dkv_multi_reduce", ptr(dkv_edge), dkv_edge.stride(0), ptr(n_uniq), max_u, ptr(csr_off), ptr(csr_edge),
         ptr(red), stream_ptr(dkv_edge.device))
    return red


def chapter_dx(dkv_edge: torch.Tensor, red: torch.Tensor, uniq, n_uniq, max_u: int, csr_off, csr_edge,
               wkv_t: torch.Tensor, out: torch.Tensor, bank_rows: bool) -> torch.Tensor:
    """Per-chapter input gradient of the K/V projection, summed over each chapter's edges:
    stored at the chapter's bank rows of ``out`` (bank_rows) or at rows c*64.. of ``out``
    ([max_u * 64][d]).  dkv_edge [E*64][2*KV] bf16, red from dkv_multi_reduce, wkv_t [d][2*KV]
    bf16."""
    N, K = wkv_t.shape
    call("moc_chapter_dx", ptr(dkv_edge), dkv_edge.stride(0), ptr(uniq), ptr(n_uniq), max_u, ptr(csr_off),
         ptr(csr_edge), ptr(red), ptr(wkv_t), N, K, L.dtype_code(out.dtype), ptr(out), out.stride(0),
         1 if bank_rows else 0, stream_ptr(dkv_edge.device))
    return out


def kv_rows_layout(kv: torch.Tensor, T: int, HK: int, Dh: int):
    """(kv_span, su, sh, st) of projection rows kv [max_u * T][2 * HK * Dh] (K columns, then V)
    for the attention entry points: block (u, hk) row t at u*T*2KV + hk*Dh + t*2KV; the span
    is what the V base (kv + HK*Dh) can still read."""
    row = 2 * HK * Dh
    return kv.numel() - HK * Dh, T * row, Dh, row


# ------------------------------------------------------------- dense projections

def rows_linear(x: torch.Tensor, w: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x W^T on the chapter GEMM over 64-row blocks of x (bf16, fp32 accumulation); w [N][K].
    ``out``: a contiguous bf16 tensor of the result's shape to write into."""
    N, K = w.shape
    x2 = x.reshape(-1, K).contiguous()
    wc = w.contiguous()
    if out is None:
        y = torch.empty(x2.shape[0], N, device=x.device, dtype=x.dtype)
    else:
        if not (out.is_contiguous() and out.dtype == x.dtype and out.numel() == x2.shape[0] * N):
            raise ValueError("rows_linear: out must be contiguous with the result's dtype and size")
        y = out.view(x2.shape[0], N)
    call("moc_rows_linear", ptr(x2), K, x2.shape[0], ptr(wc), N, K, ptr(y), N, stream_ptr(x.device))
    return y.view(*x.shape[:-1], N)


def rows_gemm_ok(x: torch.Tensor, w: torch.Tensor) -> bool:
    """Whether x W^T runs on the chapter GEMM: bf16 operands, N % 256 == 0, K % 64 == 0."""
    N, K = w.shape
    return (x.is_cuda and x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and N % 256 == 0
            and K % 64 == 0)


class _Linear(torch.autograd.Function):
    """y = x W^T (bias-free nn.Linear of the memory layer's q_proj / o_proj,
    memory_transformer/memory_attention.py:140-143, :241 and :456).  The weight gradient
    dW = dy^T x runs on the split-row MFMA kernel (the token dimension is long and the output
    small); forward and dx stay on hipBLASLt (at 8,192 x 768 x 768 it beats the chapter GEMM,
    whose 192 tiles fill one round of the chip), few rows on the few-row kernel."""

    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        if _few_rows(x, w):
            return linear_rows(x, w)
        with L.region("lib_linear_fwd"):
            return F.linear(x, w)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dx = dw = None
        if ctx.needs_input_grad[0]:
            with L.region("lib_linear_dx"):
                dx = torch.matmul(dy, w)
        if ctx.needs_input_grad[1]:
            n_out, n_in = w.shape
            dy2 = dy.reshape(-1, n_out).contiguous()
            x2 = x.reshape(-1, n_in).contiguous()
            dw = linear_wgrad(dy2, x2, w.dtype)
        return dx, dw


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return _Linear.apply(x, w)


def _few_rows(x: torch.Tensor, w: torch.Tensor) -> bool:
    K = x.shape[-1]
    return (x.is_cuda and x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and x.numel() // max(K, 1) <= 256
            and K % 128 == 0 and w.shape[0] % 16 == 0)


def linear_rows(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x W^T for at most 256 rows on the few-row kernel (bf16, fp32 accumulation)."""
    K = x.shape[-1]
    N = w.shape[0]
    x2 = x.reshape(-1, K).contiguous()
    wc = w.contiguous()
    y = torch.empty(x2.shape[0], N, device=x.device, dtype=x.dtype)
    call("moc_linear_rows", ptr(x2), x2.shape[0], K, ptr(wc), N, L.dtype_code(y.dtype), ptr(y), stream_ptr(x.device))
    return y.view(*x.shape[:-1], N)


class _LinearResidual(torch.autograd.Function):
    """out = residual + x W^T: the memory sublayer's o_proj and its residual add
    (memory_block.py:549-558, ``hidden_states = residual + mem_output``) as one GEMM with the
    residual as the accumulator input (beta = 1) when both have the output dtype."""

    @staticmethod
    def forward(ctx, x, w, residual):
        ctx.save_for_backward(x, w)
        ctx.res_dtype = residual.dtype
        n_out, n_in = w.shape
        x2 = x.reshape(-1, n_in).contiguous()
        if residual.dtype == x.dtype == w.dtype and rows_gemm_ok(x, w):
            # bf16: the residual is the GEMM's accumulator input (moc_rows_linear_residual)
            r2 = residual.reshape(-1, n_out).contiguous()
            out = torch.empty_like(r2)
            wc = w.contiguous()
            call("moc_rows_linear_residual", ptr(x2), n_in, x2.shape[0], ptr(wc), n_out, n_in, ptr(r2),
                 n_out, ptr(out), n_out, stream_ptr(x.device))
            return out.view(residual.shape)
        with L.region("lib_linear_fwd"):
            out = residual.reshape(-1, n_out) + F.linear(x2, w)
        return out.view(residual.shape)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dx = dw = dres = None
        n_out, n_in = w.shape
        dy2 = dy.reshape(-1, n_out)
        if ctx.needs_input_grad[2]:
            dres = dy
        g = dy2.to(x.dtype).contiguous()
        if ctx.needs_input_grad[0]:
            wt = w.to(x.dtype).t().contiguous()
            if rows_gemm_ok(g, wt):
                dx = rows_linear(g, wt).view(x.shape)
            else:
                with L.region("lib_linear_dx"):
                    dx = torch.matmul(g, w.to(x.dtype)).view(x.shape)
        if ctx.needs_input_grad[1]:
            dw = linear_wgrad(g, x.reshape(-1, n_in).contiguous(), w.dtype)
        return dx, dw, dres


def linear_residual(x: torch.Tensor, w: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
    return _LinearResidual.apply(x, w, residual)


class _RowNorm(torch.autograd.Function):
    """The memory sublayer's ``memory_layernorm`` (RMSNorm of memory_block.py:18-28, or
    nn.LayerNorm) on the HIP row kernels: y in ``out_dtype``; gradients for x, weight, bias."""

    @staticmethod
    def forward(ctx, x, weight, bias, norm, eps, out_dtype):
        L.require_gpu(x, weight)
        shape = x.shape
        d = shape[-1]
        x2 = x.reshape(-1, d)
        if x2.dtype not in (torch.float32, torch.bfloat16):
            x2 = x2.float()
        x2 = x2.contiguous()
        R = x2.shape[0]
        if out_dtype == torch.float32 and x2.dtype == torch.bfloat16:
            x2 = x2.float()
        w = weight.float().contiguous()
        b = bias.float().contiguous() if bias is not None else None
        dev = x2.device
        y = torch.empty(R, d, device=dev, dtype=out_dtype)
        rstd = torch.empty(R, device=dev, dtype=torch.float32)
        mean = torch.empty(R, device=dev, dtype=torch.float32) if norm == L.MOC_NORM_LAYERNORM else None
        call("moc_row_norm_fwd", norm, L.dtype_code(x2.dtype), ptr(x2), R, d, ptr(w), ptr(b), float(eps),
             L.dtype_code(out_dtype), ptr(y), ptr(mean), ptr(rstd), stream_ptr(dev))
        ctx.save_for_backward(x2, w, mean, rstd)
        ctx.cfg = (norm, shape, x.dtype, weight.dtype, None if bias is None else bias.dtype)
        return y.view(*shape[:-1], d)

    @staticmethod
    def backward(ctx, dy):
        x2, w, mean, rstd = ctx.saved_tensors
        norm, shape, x_dtype, w_dtype, b_dtype = ctx.cfg
        R, d = x2.shape
        dev = x2.device
        dy2 = dy.reshape(R, d)
        if x2.dtype == torch.bfloat16:
            dy2 = dy2.to(torch.bfloat16)
        elif dy2.dtype not in (torch.float32, torch.bfloat16):
            dy2 = dy2.float()
        dy2 = dy2.contiguous()
        dx = torch.empty(R, d, device=dev, dtype=x2.dtype)
        dwb = torch.empty(2, d, device=dev, dtype=torch.float32)
        ws_bytes = L.query("moc_row_norm_bwd_workspace", R, d)
        ws = torch.empty(max(1, ws_bytes // 4), device=dev, dtype=torch.float32)
        call("moc_row_norm_bwd", norm, L.dtype_code(x2.dtype), ptr(x2), R, d, ptr(w), ptr(mean), ptr(rstd),
             L.dtype_code(dy2.dtype), ptr(dy2), L.dtype_code(dx.dtype), ptr(dx), ptr(dwb), ptr(ws), ws_bytes,
             stream_ptr(dev))
        dw = dwb[0].to(w_dtype) if ctx.needs_input_grad[1] else None
        db = dwb[1].to(b_dtype) if (b_dtype is not None and ctx.needs_input_grad[2]) else None
        return dx.view(shape).to(x_dtype), dw, db, None, None, None


def row_norm(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], eps: float, norm: str = "rms",
             out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """RMSNorm (``norm="rms"``) or LayerNorm (``"layer"``) over the last dim, output in
    ``out_dtype`` (default: x's dtype)."""
    code = {"rms": L.MOC_NORM_RMS, "layer": L.MOC_NORM_LAYERNORM}.get(norm)
    if code is None:
        raise ValueError(f"norm must be 'rms' or 'layer', got {norm!r}")
    od = x.dtype if out_dtype is None else out_dtype
    if od not in (torch.float32, torch.bfloat16):
        raise ValueError(f"row_norm outputs float32 or bfloat16, got {od}")
    return _RowNorm.apply(x, weight, bias, code, float(eps), od)


class _NormLinear(torch.autograd.Function):
    """q_proj(memory_layernorm(x)) of the memory sublayer (memory_block.py:549-558 with
    memory_attention.py:241) as one GEMM: the norm weight folded into the projection weight
    (``moc_norm_fold_weight``) and the row statistics taken inside the GEMM
    (``moc_rows_linear_norm``), so the normalised rows are never written in the forward.
    Backward: d(normalised rows) = dy W on the chapter GEMM, the norm's backward
    (``moc_row_norm_bwd``) from x and the statistics the GEMM wrote, and dW = dy^T norm(x) with
    the normalised rows recomputed here (the only place they are materialised)."""

    @staticmethod
    def forward(ctx, x, weight, bias, w, norm, eps):
        N, K = w.shape
        x2 = x.reshape(-1, K).contiguous()
        R = x2.shape[0]
        dev = x.device
        st = stream_ptr(dev)
        g = weight.float().contiguous()
        b = bias.float().contiguous() if bias is not None else None
        wc = w.contiguous()
        wf = torch.empty_like(wc)
        ln = norm == L.MOC_NORM_LAYERNORM
        u = torch.empty(N, device=dev, dtype=torch.float32) if ln else None
        v = torch.empty(N, device=dev, dtype=torch.float32) if ln else None
        call("moc_norm_fold_weight", ptr(wc), N, K, ptr(g), ptr(b), ptr(wf), ptr(u), ptr(v), st)
        y = torch.empty(R, N, device=dev, dtype=torch.bfloat16)
        rstd = torch.empty(R, device=dev, dtype=torch.float32)
        mean = torch.empty(R, device=dev, dtype=torch.float32) if ln else None
        call("moc_rows_linear_norm", ptr(x2), K, R, ptr(wf), N, K, norm, float(eps), ptr(u), ptr(v), ptr(y), N,
             ptr(mean), ptr(rstd), st)
        ctx.save_for_backward(x2, g, b, wc, mean, rstd)
        ctx.cfg = (norm, float(eps), x.shape, weight.dtype, None if bias is None else bias.dtype)
        return y.view(*x.shape[:-1], N)

    @staticmethod
    def backward(ctx, dy):
        x2, g, b, w, mean, rstd = ctx.saved_tensors
        norm, eps, shape, w_dtype, b_dtype = ctx.cfg
        R, K = x2.shape
        N = w.shape[0]
        dev = x2.device
        st = stream_ptr(dev)
        dy2 = dy.reshape(R, N).to(torch.bfloat16).contiguous()
        dx = dg = db = dw = None
        if ctx.needs_input_grad[0] or ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
            dxn = rows_linear(dy2, w.t().contiguous()) if K % 256 == 0 and N % 64 == 0 else torch.matmul(dy2, w)
            dxr = torch.empty(R, K, device=dev, dtype=torch.bfloat16)
            dwb = torch.empty(2, K, device=dev, dtype=torch.float32)
            ws_bytes = L.query("moc_row_norm_bwd_workspace", R, K)
            ws = torch.empty(max(1, ws_bytes // 4), device=dev, dtype=torch.float32)
            call("moc_row_norm_bwd", norm, L.MOC_BF16, ptr(x2), R, K, ptr(g), ptr(mean), ptr(rstd), L.MOC_BF16,
                 ptr(dxn), L.MOC_BF16, ptr(dxr), ptr(dwb), ptr(ws), ws_bytes, st)
            dx = dxr.view(shape)
            dg = dwb[0].to(w_dtype) if ctx.needs_input_grad[1] else None
            db = dwb[1].to(b_dtype) if (b_dtype is not None and ctx.needs_input_grad[2]) else None
        if ctx.needs_input_grad[3]:
            xn = torch.empty(R, K, device=dev, dtype=torch.bfloat16)
            m2 = torch.empty(R, device=dev, dtype=torch.float32) if norm == L.MOC_NORM_LAYERNORM else None
            r2 = torch.empty(R, device=dev, dtype=torch.float32)
            call("moc_row_norm_fwd", norm, L.MOC_BF16, ptr(x2), R, K, ptr(g), ptr(b), eps, L.MOC_BF16, ptr(xn),
                 ptr(m2), ptr(r2), st)
            dw = linear_wgrad(dy2, xn, w.dtype)
        return dx, dg, db, dw, None, None


def norm_linear_supported(x: torch.Tensor, w: torch.Tensor) -> bool:
    """Shapes and dtypes the fused norm + projection takes (bf16 rows and weight, N a multiple
    of 256, K of 64, on a ROCm device)."""
    N, K = w.shape
    return (x.is_cuda and x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and x.shape[-1] == K
            and N % 256 == 0 and K % 64 == 0)


def norm_linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], eps: float, norm: str,
                w: torch.Tensor) -> torch.Tensor:
    """``norm(x) W^T`` with norm = RMSNorm (``"rms"``) or LayerNorm (``"layer"``) over the last
    dim: one fused GEMM where ``norm_linear_supported``, else the norm kernel then the projection."""
    code = {"rms": L.MOC_NORM_RMS, "layer": L.MOC_NORM_LAYERNORM}.get(norm)
    if code is None:
        raise ValueError(f"norm must be 'rms' or 'layer', got {norm!r}")
    if norm_linear_supported(x, w):
        return _NormLinear.apply(x, weight, bias if code == L.MOC_NORM_LAYERNORM else None, w, code, float(eps))
    return linear(row_norm(x, weight, bias, eps, norm, w.dtype), w)


def linear_wgrad(dy: torch.Tensor, x: torch.Tensor, out_dtype: torch.dtype,
                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """dW = dy^T x for dy [R][N], x [R][K] (row-major, contiguous): the split-row MFMA
    kernel for bf16 dy (N, K multiples of 8), a plain GEMM otherwise.  ``out``: a [N][K]
    tensor of out_dtype to write (allocated here when None)."""
    R, N = dy.shape
    K = x.shape[1]
    dw = torch.empty(N, K, device=dy.device, dtype=out_dtype) if out is None else out
    if (dy.dtype == torch.bfloat16 and x.dtype in (torch.bfloat16, torch.float32) and dy.is_cuda and N % 8 == 0
            and K % 8 == 0 and out_dtype in (torch.float32, torch.bfloat16)):
        ws = torch.empty(L.query("moc_linear_wgrad_workspace", R, N, K) // 4, device=dy.device, dtype=torch.float32)
        call("moc_linear_wgrad", ptr(dy), ptr(x), L.dtype_code(x.dtype), R, N, K, ptr(ws), ws.numel() * 4,
             L.dtype_code(out_dtype), ptr(dw), stream_ptr(dy.device))
        return dw
    dw.copy_(torch.matmul(dy.t().to(x.dtype), x))
    return dw


# ------------------------------------------------------------- routed attention (A)

_ATTN_SAVED = ("q", "bank", "wkv", "om", "out", "lse", "kv", "mean", "rstd", "uniq", "n_uniq", "edge_u", "csr_off",
               "csr_edge")


def _tiny_chapters(max_u: int, T: int, d: int, KV: int) -> bool:
    """At most 256 rows of distinct chapters with the few-row kernel's shapes (d, 2 KV multiples
    of 128): the K/V projection and its input gradient run on moc_linear_rows."""
    return max_u * T <= 256 and d % 128 == 0 and (2 * KV) % 128 == 0


def routed_attn_forward(q, bank, wk, wv, omega, idx_star, num_chapters, T, norm, eps, HK, wkv=None):
    """Forward body of the sequence-routed attention (plan, gather + K/V projection, joint
    attention): returns (out, saved tensors in _ATTN_SAVED order, cfg).  ``wkv``: the packed
    bf16 [Wk; Wv] when the caller already has it (its pack then stays off this stream)."""
    L.require_gpu(q, bank, wk, wv, omega, idx_star)
    dtype = q.dtype
    bank_dtype = bank.dtype
    B, Lq, H, Dh = q.shape
    NS = idx_star.shape[1]
    q = q.contiguous()
    # a bank stepped by BankAdamW: its plan's chapters are brought to the last step before
    # they are read, and the forward kernels read its mirror when it keeps one
    opt = getattr(bank, "_moc_bank_opt", None)
    plan = chapter_plan(idx_star, num_chapters)
    if opt is not None:
        opt.catch_up(plan.uniq, plan.n_uniq, plan.max_u)
        bank = opt.read_view(dtype)
    bank = bank.contiguous()
    mean = rstd = None
    if norm != L.MOC_NORM_NONE:
        mean, rstd = row_stats(bank, plan, T, norm, eps)
    # K / V of the plan's chapters as projection rows [max_u * T][K | V]; the attention
    # kernels read (chapter, kv head) blocks of it through strides
    KV = HK * Dh
    d = bank.shape[1]
    if dtype == torch.bfloat16 and T == 64 and (2 * KV) % 256 == 0 and d % 64 == 0:
        # bf16: the chapter GEMM, gathering bank rows straight into its operand tiles (a
        # normalised or f32 bank is gathered into bf16 rows first)
        if wkv is None:
            wkv, _ = weight_pack(wk, wv)
        if _tiny_chapters(plan.max_u, T, d, KV):
            # a few chapters (the token path's shared chapters): their rows gathered, then the
            # few-row kernel, whose loads go out in one round (a persistent GEMM would walk the
            # whole K dimension on one tile)
            X = torch.empty(plan.max_u * T, d, device=q.device, dtype=dtype)
            call("moc_gather_rows", L.dtype_code(dtype), ptr(bank), L.dtype_code(bank.dtype), d, T,
                 ptr(plan.uniq), ptr(plan.n_uniq), plan.max_u, ptr(mean), ptr(rstd), ptr(X), stream_ptr(q.device))
            kv = linear_rows(X, wkv)
            del X
        elif norm == L.MOC_NORM_NONE and bank.dtype == torch.bfloat16:
            kv = chapter_project(bank, plan, wkv, gather=True)
        else:
            X = torch.empty(plan.max_u * T, d, device=q.device, dtype=dtype)
            call("moc_gather_rows", L.dtype_code(dtype), ptr(bank), L.dtype_code(bank.dtype), d, T,
                 ptr(plan.uniq), ptr(plan.n_uniq), plan.max_u, ptr(mean), ptr(rstd), ptr(X), stream_ptr(q.device))
            kv = chapter_project(X, plan, wkv, gather=False)
            del X
    else:
        wkv = torch.cat([wk, wv], 0).to(dtype).contiguous()
        X = torch.empty(plan.max_u * T, d, device=q.device, dtype=dtype)
        call("moc_gather_rows", L.dtype_code(dtype), ptr(bank), L.dtype_code(bank.dtype), d, T,
             ptr(plan.uniq), ptr(plan.n_uniq), plan.max_u, ptr(mean), ptr(rstd), ptr(X), stream_ptr(q.device))
        with L.region("lib_kv_project_gemm"):
            kv = F.linear(X, wkv)
        del X
    kvl = kv_rows_layout(kv, T, HK, Dh)
    om = omega.float().contiguous()
    out = torch.empty(B, Lq, H, Dh, device=q.device, dtype=dtype)
    Lp = (Lq + 127) // 128 * 128
    lse = torch.empty(B, H, Lp, device=q.device, dtype=torch.float32)
    call("moc_xattn_fwd", L.dtype_code(dtype), ptr(q), ptr(kv), ptr(kv) + KV * kv.element_size(), *kvl,
         ptr(plan.edge_u), ptr(om), B, Lq, H, HK, Dh, T, NS, float(Dh) ** -0.5, ptr(out), ptr(lse),
         stream_ptr(q.device))
    saved = (q, bank, wkv, om, out, lse, kv, mean, rstd, plan.uniq, plan.n_uniq, plan.edge_u, plan.csr_off,
             plan.csr_edge)
    cfg = (num_chapters, T, norm, eps, HK, plan.max_u, wk.dtype, wv.dtype, bank_dtype)
    return out, saved, cfg


def routed_attn_backward(saved, cfg, dout, needs, row_grad=None, after_dq=None, after_dkv=None):
    """Backward body of the sequence-routed attention.  ``needs`` = (q, bank, wk, wv, omega)
    input-gradient flags.  Returns (dq, dbank, dwk, dwv, dom_part) with dom_part f32
    [B * NS, HK] (d omega per (edge, kv head); d omega = its sum over kv heads).  The hooks run
    on the host right after the dQ launch (``after_dq(dq)``) and after the dK/dV launch
    (``after_dkv(dom_part)``): callers fork work that needs only those onto other streams."""
    (q, bank, wkv, om, out, lse, kv, mean, rstd, uniq, n_uniq, edge_u, csr_off, csr_edge) = saved
    C, T, norm, eps, HK, max_u, wk_dtype, wv_dtype, bank_dtype = cfg
    dtype = q.dtype
    dt = L.dtype_code(dtype)
    B, Lq, H, Dh = q.shape
    NS = om.shape[1]
    KV = HK * Dh
    d = bank.shape[1]
    dev = q.device
    st = stream_ptr(dev)
    scale = float(Dh) ** -0.5
    _need_q, need_bank, need_wk, need_wv, _need_om = needs
    dout = dout.to(dtype).contiguous()
    Lp = lse.shape[2]
    delta = torch.empty(B, H, Lp, device=dev, dtype=torch.float32)   # written by the dQ kernel
    # the dense bank gradient's zeros are written beside the dQ and dK/dV kernels
    dbank_zero = None
    if dtype == torch.bfloat16 and need_bank and row_grad is None:
        dbank_zero = zeros_beside(bank.shape, bank.dtype, dev)
    dq = torch.empty_like(q)
    kvl = kv_rows_layout(kv, T, HK, Dh)
    vptr = ptr(kv) + KV * kv.element_size()
    call("moc_xattn_bwd_dq_delta", dt, ptr(q), ptr(kv), vptr, *kvl, ptr(edge_u), ptr(om), ptr(out),
         ptr(dout), ptr(lse), ptr(delta), B, Lq, H, HK, Dh, T, NS, scale, ptr(dq), st)
    if after_dq is not None:
        after_dq(dq)
    dkv_edge = torch.empty(B * NS * T, 2 * KV, device=dev, dtype=dtype)
    dom_part = torch.empty(B * NS, HK, device=dev, dtype=torch.float32)   # every entry written
    call("moc_xattn_bwd_dkv", dt, ptr(q), ptr(dout), ptr(kv), vptr, *kvl, ptr(edge_u), ptr(om),
         ptr(lse), ptr(delta), B, Lq, H, HK, Dh, T, NS, scale, ptr(dkv_edge), ptr(dom_part), st)
    if after_dkv is not None:
        after_dkv(dom_part)
    dbank = dwk = dwv = None
    E = B * NS
    if dtype == torch.bfloat16:
        # the chapter GEMMs read a chapter's dK|dV rows in place when one edge selected it and
        # from `red` (the edges' sum, written once here) when several did
        tiled = T == 64 and d % 256 == 0 and (2 * KV) % 256 == 0
        red = None
        if tiled and (need_bank or need_wk or need_wv):
            red = torch.empty(max_u * T, 2 * KV, device=dev, dtype=torch.bfloat16)
            call("moc_dkv_multi_reduce", ptr(dkv_edge), 2 * KV, ptr(n_uniq), max_u, ptr(csr_off), ptr(csr_edge),
                 ptr(red), st)
        dwkv = None
        if need_wk or need_wv:
            out_dt = torch.float32 if torch.float32 in (wk_dtype, wv_dtype) else dtype
            dwkv = torch.empty(2 * KV, d, device=dev, dtype=out_dt)
            if tiled:
                # dW = sum over distinct chapters of dK|dV_c^T X_c (bank rows gathered by
                # the kernel; a normalised or f32 bank is gathered into bf16 rows first)
                ws_bytes = L.query("moc_chapter_wgrad_workspace", 2 * KV, d, max_u)
                ws = torch.empty(ws_bytes // 4, device=dev, dtype=torch.float32)
                if norm == L.MOC_NORM_NONE and bank.dtype == torch.bfloat16:
                    xs, gather = bank, 1
                else:
                    xs = torch.empty(max_u * T, d, device=dev, dtype=torch.bfloat16)
                    call("moc_gather_rows", L.MOC_BF16, ptr(bank), L.dtype_code(bank.dtype), d, T,
                         ptr(uniq), ptr(n_uniq), max_u, ptr(mean), ptr(rstd), ptr(xs), st)
                    gather = 0
                call("moc_chapter_wgrad", ptr(dkv_edge), 2 * KV, ptr(red), ptr(xs), xs.stride(0), gather,
                     ptr(uniq), ptr(n_uniq), max_u, ptr(csr_off), ptr(csr_edge), 2 * KV, d, ptr(ws),
                     ws_bytes, L.dtype_code(out_dt), ptr(dwkv), st)
            else:
                # per-edge rows paired with their chapter's bank rows (no per-chapter sums)
                ws = torch.empty(L.query("moc_kv_wgrad_workspace", 2 * KV, d, E) // 4, device=dev,
                                 dtype=torch.float32)
                call("moc_kv_wgrad", ptr(dkv_edge), ptr(bank), L.dtype_code(bank.dtype), d, T,
                     ptr(uniq), ptr(n_uniq), ptr(edge_u), E, ptr(mean), ptr(rstd), 2 * KV, ptr(ws),
                     ws.numel() * 4, L.dtype_code(out_dt), ptr(dwkv), st)
        if need_bank and not tiled:
            # shapes outside the chapter GEMM's tiling: per-edge dX on the library GEMM,
            # summed per chapter by the scatter
            dX = torch.matmul(dkv_edge, wkv)  # rows of skipped edges are never read
            if row_grad is not None:
                row_grad.accumulate(dX, bank, uniq, n_uniq, max_u, csr_off, csr_edge, mean, rstd, norm)
            else:
                dbank, filled = dbank_zero
                if filled is not None:
                    torch.cuda.current_stream(dev).wait_event(filled)
                call("moc_bank_scatter", L.dtype_code(dX.dtype), ptr(dX), ptr(bank), L.dtype_code(bank.dtype),
                     d, T, ptr(uniq), ptr(n_uniq), max_u, ptr(csr_off), ptr(csr_edge), ptr(mean), ptr(rstd),
                     norm, ptr(dbank), st)
                dbank = dbank.to(bank_dtype)
        elif need_bank:
            # dX per distinct chapter (edges summed) on the chapter GEMM; with a plain bank it
            # is stored straight into the chapter's rows of the dense gradient
            _, wkv_t = weight_pack(wkv[:KV], wkv[KV:], rows=False, transposed=True)
            if _tiny_chapters(max_u, T, d, KV):
                # a few chapters: the edges' rows summed per chapter, dX on the few-row kernel
                # (fp32 out), then the scatter into the bank gradient
                dkv_c = torch.empty(max_u * T, 2 * KV, device=dev, dtype=torch.bfloat16)
                call("moc_dkv_reduce", L.MOC_BF16, ptr(dkv_edge), ptr(n_uniq), ptr(csr_off), ptr(csr_edge), max_u,
                     2 * KV, ptr(dkv_c), st)
                dXc = torch.empty(max_u * T, d, device=dev, dtype=torch.float32)
                call("moc_linear_rows", ptr(dkv_c), max_u * T, 2 * KV, ptr(wkv_t), d, L.MOC_F32, ptr(dXc), st)
                if row_grad is not None:
                    row_grad.accumulate(dXc, bank, uniq, n_uniq, max_u, None, None, mean, rstd, norm)
                else:
                    dbank, filled = dbank_zero
                    if filled is not None:
                        torch.cuda.current_stream(dev).wait_event(filled)
                    call("moc_bank_scatter", L.MOC_F32, ptr(dXc), ptr(bank), L.dtype_code(bank.dtype), d, T,
                         ptr(uniq), ptr(n_uniq), max_u, None, None, ptr(mean), ptr(rstd), norm, ptr(dbank), st)
                    dbank = dbank.to(bank_dtype)
            elif row_grad is None and norm == L.MOC_NORM_NONE:
                dbank, filled = dbank_zero
                if filled is not None:
                    torch.cuda.current_stream(dev).wait_event(filled)
                chapter_dx(dkv_edge, red, uniq, n_uniq, max_u, csr_off, csr_edge, wkv_t, dbank, bank_rows=True)
                dbank = dbank.to(bank_dtype)   # the bank read may be a mirror of another dtype
            else:
                dXc = torch.empty(max_u * T, d, device=dev, dtype=torch.float32)
                chapter_dx(dkv_edge, red, uniq, n_uniq, max_u, csr_off, csr_edge, wkv_t, dXc, bank_rows=False)
                if row_grad is not None:
                    row_grad.accumulate(dXc, bank, uniq, n_uniq, max_u, None, None, mean, rstd, norm)
                else:
                    dbank, filled = dbank_zero
                    if filled is not None:
                        torch.cuda.current_stream(dev).wait_event(filled)
                    call("moc_bank_scatter", L.dtype_code(dXc.dtype), ptr(dXc), ptr(bank),
                         L.dtype_code(bank.dtype), d, T, ptr(uniq), ptr(n_uniq), max_u, None, None, ptr(mean),
                         ptr(rstd), norm, ptr(dbank), st)
                    dbank = dbank.to(bank_dtype)
        if dwkv is not None:
            dwk = dwkv[:KV].to(wk_dtype) if need_wk else None
            dwv = dwkv[KV:].to(wv_dtype) if need_wv else None
        return dq, dbank, dwk, dwv, dom_part
    # fp32: sum per distinct chapter first, then library GEMMs
    dkv = torch.empty(max_u * T, 2 * KV, device=dev, dtype=dtype)
    call("moc_dkv_reduce", dt, ptr(dkv_edge), ptr(n_uniq), ptr(csr_off), ptr(csr_edge), max_u, 2 * KV, ptr(dkv),
         st)
    if need_wk or need_wv:
        X = torch.empty(max_u * T, d, device=dev, dtype=dtype)
        call("moc_gather_rows", dt, ptr(bank), L.dtype_code(bank.dtype), d, T, ptr(uniq), ptr(n_uniq),
             max_u, ptr(mean), ptr(rstd), ptr(X), st)
        dwkv = torch.matmul(dkv.t(), X)
        dwk = dwkv[:KV].to(wk_dtype) if need_wk else None
        dwv = dwkv[KV:].to(wv_dtype) if need_wv else None
    if need_bank:
        dX = torch.matmul(dkv, wkv)
        if row_grad is not None:
            row_grad.accumulate(dX, bank, uniq, n_uniq, max_u, None, None, mean, rstd, norm)
        else:
            dbank = torch.zeros(bank.shape, device=dev, dtype=bank.dtype)
            call("moc_bank_scatter", L.dtype_code(dX.dtype), ptr(dX), ptr(bank), L.dtype_code(bank.dtype), d,
                 T, ptr(uniq), ptr(n_uniq), max_u, None, None, ptr(mean), ptr(rstd), norm, ptr(dbank), st)
            dbank = dbank.to(bank_dtype)
    return dq, dbank, dwk, dwv, dom_part




class _RoutedAttention(torch.autograd.Function):
    """Gather + K/V projection + joint routed attention (sequence level).

    Inputs: q (B, L, H, Dh) [compute dtype]; bank (N_m, d); wk/wv (HK*Dh, d);
    omega (B, NS) fp32 chapter weights; idx_star (B, NS) chapter ids.
    Output: attention output (B, L, H, Dh) before o_proj."""

    @staticmethod
    def forward(ctx, q, bank, wk, wv, omega, idx_star, num_chapters, T, norm, eps, HK):
        # a bank with a RowSparseBankGrad receives its gradient rows there instead of a dense gradient
        ctx.row_grad = getattr(bank, "_moc_row_grad", None)
        out, saved, cfg = routed_attn_forward(q, bank, wk, wv, omega, idx_star, num_chapters, T, norm, eps, HK)
        ctx.save_for_backward(*saved)
        ctx.cfg = cfg
        return out

    @staticmethod
    def backward(ctx, dout):
        needs = tuple(ctx.needs_input_grad[:5])
        dq, dbank, dwk, dwv, dom_part = routed_attn_backward(ctx.saved_tensors, ctx.cfg, dout, needs,
                                                              row_grad=ctx.row_grad)
        domega = None
        if ctx.needs_input_grad[4]:
            B, NS = ctx.saved_tensors[3].shape
            domega = dom_part.sum(-1).view(B, NS)
        return dq, dbank, dwk, dwv, domega, None, None, None, None, None, None


_SIDE_STREAMS: dict = {}


def _side_stream(dev: torch.device, name: str = "fill") -> torch.cuda.Stream:
    """A second stream (default priority) per device and purpose for work that runs beside
    the main sequence of kernels."""
    key = (dev.type, dev.index, name)
    s = _SIDE_STREAMS.get(key)
    if s is None:
        s = _SIDE_STREAMS[key] = torch.cuda.Stream(device=dev)
    return s


def zeros_beside(shape, dtype: torch.dtype, dev: torch.device, workgroups: Optional[int] = None):
    """A zero-filled tensor whose fill (moc_fill_zero, one single-wave workgroup per CU) runs
    on a side stream, so that it overlaps the compute-bound kernels queued next on the
    current stream.  Returns (tensor, event); the current stream must wait on the event
    before it touches the tensor (event None: filled in order on the current stream)."""
    t = torch.empty(shape, device=dev, dtype=dtype)
    nbytes = t.numel() * t.element_size()
    if nbytes % 16 or t.data_ptr() % 16:
        t.zero_()
        return t, None
    main = torch.cuda.current_stream(dev)
    side = _side_stream(dev)
    side.wait_stream(main)
    if workgroups is None:
        workgroups = torch.cuda.get_device_properties(dev).multi_processor_count
    call("moc_fill_zero", ptr(t), nbytes, int(workgroups), side.cuda_stream)
    t.record_stream(side)
    ev = torch.cuda.Event()
    ev.record(side)
    return t, ev


def sub_chapters(bank, omega, idx_star, num_chapters: int, tokens_per_chapter: int):
    """Chapters of T = 64 m bank rows as m consecutive 64-row chapters (the kernels' chapter
    tile): chapter c becomes sub-chapters m c .. m c + m - 1 with c's weight.  The joint softmax
    over a sequence's selected keys, the keys' order and the gradients are unchanged (the
    weight's gradient is the sum of its sub-chapters', by autograd of the repeat); ids outside
    [0, C) stay outside [0, m C).  Returns (omega, idx_star, num_chapters) for T = 64."""
    T = int(tokens_per_chapter)
    if T <= 0 or T % 64:
        raise ValueError(f"tokens_per_chapter must be a positive multiple of 64 for the HIP kernels, got {T}")
    m = T // 64
    if m == 1:
        return omega, idx_star, int(num_chapters)
    for attr in ("_moc_bank_opt", "_moc_row_grad"):
        if getattr(bank, attr, None) is not None:
            raise NotImplementedError(f"tokens_per_chapter {T}: a bank with row-sparse gradients or BankAdamW "
                                      "needs 64-row chapters")
    sub = torch.arange(m, device=idx_star.device, dtype=torch.int64)
    idx = (idx_star.long().unsqueeze(-1) * m + sub).flatten(-2).to(idx_star.dtype)
    return omega.repeat_interleave(m, dim=-1), idx, int(num_chapters) * m


def routed_attention(q, bank, wk, wv, omega, idx_star, *, num_chapters: int, tokens_per_chapter: int,
                     norm_type: Optional[str] = None, eps: float = 1e-6, num_kv_heads: Optional[int] = None):
    HK = q.shape[2] if num_kv_heads is None else int(num_kv_heads)
    omega, idx_star, num_chapters = sub_chapters(bank, omega, idx_star, num_chapters, tokens_per_chapter)
    return _RoutedAttention.apply(q, bank, wk, wv, omega, idx_star, int(num_chapters), 64,
                                  norm_code(norm_type), float(eps), HK)


@torch.no_grad()
def routed_attention_weights(q, bank, wk, wv, omega, idx_star, *, num_chapters: int, tokens_per_chapter: int,
                             norm_type: Optional[str] = None, eps: float = 1e-6,
                             num_kv_heads: Optional[int] = None) -> torch.Tensor:
    """softmax(q k^T * scale) of the sequence-routed attention, (B, H, L, NS * T) in q's dtype
    (memory_attention.py:437-447 on the omega-weighted gathered memory): the forward's K and row
    log-sum-exp, then moc_xattn_weights."""
    HK = q.shape[2] if num_kv_heads is None else int(num_kv_heads)
    omega, idx_star, num_chapters = sub_chapters(bank, omega, idx_star, num_chapters, tokens_per_chapter)
    T = 64
    _, saved, _ = routed_attn_forward(q, bank, wk, wv, omega, idx_star, int(num_chapters), T, norm_code(norm_type),
                                      float(eps), HK)
    qc, _, _, om, _, lse, kv, *_rest = saved
    edge_u = saved[11]
    B, Lq, H, Dh = qc.shape
    NS = om.shape[1]
    P = torch.empty(B, H, Lq, NS * T, device=q.device, dtype=qc.dtype)
    call("moc_xattn_weights", L.dtype_code(qc.dtype), ptr(qc), ptr(kv), *kv_rows_layout(kv, T, HK, Dh), ptr(edge_u),
         ptr(om), B, Lq, H, HK, Dh, T, NS, float(Dh) ** -0.5, ptr(lse), ptr(P), stream_ptr(q.device))
    return P


class _TokenRouterLinear(torch.autograd.Function):
    """logits = x W^T + b for per-token routing (router.py:294, ``self.router(hidden_states)``).

    The GEMM operands are in the activation dtype (bf16 activations round W to bf16, the
    operand precision of the reference under autocast) and accumulate in fp32; the logits stay
    fp32 (not rounded to bf16 as under autocast) so that the top-k selection sees distinct
    values.  bf16: the chapter GEMM with the bias in its epilogue (moc_rows_linear_f32, any
    number of chapters).  Backward: dx = dlogits W in the activation dtype, dW = dlogits^T x and
    db = sum dlogits in fp32; for bf16 the logit gradient is rounded once into a bf16 copy whose
    rows are padded with zeros to a multiple of 256 chapters, so that both products run on the
    chapter kernels (dx on the rows GEMM with the zero-padded W^T, dW on the split-row weight
    gradient, its padded rows dropped).  fp32 activations stay on library GEMMs."""

    @staticmethod
    def forward(ctx, x, W, b):
        Wc = W.to(x.dtype).contiguous()
        R, K = x.shape
        C = Wc.shape[0]
        if x.dtype == torch.bfloat16 and K % 64 == 0:
            y = torch.empty(R, C, device=x.device, dtype=torch.float32)
            bias = None if b is None else b.float().contiguous()
            call("moc_rows_linear_f32", ptr(x), K, R, ptr(Wc), C, K, None if bias is None else ptr(bias), ptr(y), C,
                 stream_ptr(x.device))
        elif b is None:
            y = torch.mm(x, Wc.t()) if x.dtype == torch.float32 else torch.mm(x, Wc.t(), out_dtype=torch.float32)
        elif x.dtype == torch.float32:
            y = torch.addmm(b.float(), x, Wc.t())
        else:
            y = torch.addmm(b.float(), x, Wc.t(), out_dtype=torch.float32)
        ctx.save_for_backward(x, Wc)
        ctx.meta = (W.dtype, None if b is None else b.dtype)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, Wc = ctx.saved_tensors
        w_dtype, b_dtype = ctx.meta
        dy = dy.contiguous()
        R, K = x.shape
        C = Wc.shape[0]
        dx = dW = db = None
        need_db = b_dtype is not None and ctx.needs_input_grad[2]
        if x.dtype == torch.bfloat16 and K % 256 == 0:
            # one pass over the fp32 logit gradient: the zero-padded bf16 operand and the bias
            # gradient's column sums (moc_logit_grad_pack)
            Cp = (C + 255) // 256 * 256
            dyp = torch.empty(R, Cp, device=dy.device, dtype=torch.bfloat16)
            db32 = torch.empty(C, device=dy.device, dtype=torch.float32) if need_db else None
            ws_bytes = L.query("moc_logit_grad_pack_workspace", R, C) if need_db else 0
            ws = torch.empty(max(1, ws_bytes // 4), device=dy.device, dtype=torch.float32) if need_db else None
            call("moc_logit_grad_pack", ptr(dy), R, C, Cp, ptr(dyp), ptr(db32), ptr(ws), ws_bytes,
                 stream_ptr(dy.device))
            if need_db:
                db = db32.to(b_dtype)
            if ctx.needs_input_grad[0]:
                # W^T with its chapter columns zero-padded to Cp, in one transposing pass
                wt = torch.empty(K, Cp, device=dy.device, dtype=torch.bfloat16)
                call("moc_weight_transpose", ptr(Wc), L.dtype_code(Wc.dtype), C, K, ptr(wt), Cp,
                     stream_ptr(dy.device))
                dx = rows_linear(dyp, wt)
            if ctx.needs_input_grad[1]:
                dW = linear_wgrad(dyp, x, torch.float32)[:C].to(w_dtype)
        else:
            dyc = dy if x.dtype == torch.float32 else dy.to(x.dtype)
            if ctx.needs_input_grad[0]:
                dx = torch.mm(dyc, Wc)
            if ctx.needs_input_grad[1]:
                if x.dtype == torch.float32:
                    dW = torch.mm(dyc.t(), x)
                else:
                    dW = torch.mm(dyc.t(), x, out_dtype=torch.float32)
                dW = dW.to(w_dtype)
        if need_db and db is None:
            db = col_sum(dy).to(b_dtype)
        return dx, dW, db


class _RouterLosses(torch.autograd.Function):
    """The router's auxiliary losses (router.py:197-260) in one pass over the logits:
    returns f32 [4] = (load_balance, auxiliary, z_loss, entropy); the gradient flows to the
    logits (the selection counts are constants, as the reference's one-hot is)."""

    @staticmethod
    def forward(ctx, logits: torch.Tensor, idx: torch.Tensor, num_chapters: int):
        L.require_gpu(logits, idx)
        z = logits.reshape(-1, logits.shape[-1]).float().contiguous()
        R, C = z.shape
        if C != int(num_chapters):
            raise ValueError(f"logits have {C} chapters, expected {num_chapters}")
        sel = idx.reshape(R, -1).to(torch.int32).contiguous()
        k = sel.shape[1]
        dev = z.device
        row_lse = torch.empty(R, device=dev, dtype=torch.float32)
        coef = torch.empty(C, 2, device=dev, dtype=torch.float32)
        counts = torch.empty(C, device=dev, dtype=torch.int32)
        losses = torch.empty(4, device=dev, dtype=torch.float32)
        ws_bytes = L.query("moc_router_losses_workspace", R, C)
        ws = torch.empty(ws_bytes // 4, device=dev, dtype=torch.float32)
        call("moc_router_losses", ptr(z), R, C, ptr(sel) if k else None, k, ptr(row_lse), ptr(coef), ptr(counts),
             ptr(losses), ptr(ws), ws_bytes, stream_ptr(dev))
        ctx.save_for_backward(z, row_lse, coef)
        ctx.shape, ctx.dtype = logits.shape, logits.dtype
        return losses

    @staticmethod
    def backward(ctx, dlosses):
        z, row_lse, coef = ctx.saved_tensors
        R, C = z.shape
        dz = torch.empty_like(z)
        g = dlosses.float().contiguous()
        call("moc_router_losses_bwd", ptr(z), R, C, ptr(row_lse), ptr(coef), ptr(g), ptr(dz), stream_ptr(z.device))
        return dz.view(ctx.shape).to(ctx.dtype), None, None


ROUTER_LOSS_NAMES = ("load_balance", "auxiliary", "z_loss", "entropy")


def router_losses(logits: torch.Tensor, idx: torch.Tensor, num_chapters: int):
    """Dict of the four router losses (scalar tensors) on the fused kernels."""
    v = _RouterLosses.apply(logits, idx, int(num_chapters))
    return {n: v[i] for i, n in enumerate(ROUTER_LOSS_NAMES)}


def col_sum(x: torch.Tensor) -> torch.Tensor:
    """Column sums (fp32) of a 2-D fp32 / bf16 matrix on the router's pooling kernels
    (fixed-order split-row partials, deterministic)."""
    x = x.contiguous()
    R, C = x.shape
    out = torch.empty(C, device=x.device, dtype=torch.float32)
    if R == 0:
        return out.zero_()
    ones = torch.ones(R, device=x.device, dtype=torch.float32)
    ws_bytes = L.query("moc_router_pool_workspace", 1, R, C)
    ws = torch.empty(max(1, ws_bytes // 4), device=x.device, dtype=torch.float32)
    call("moc_router_pool", ptr(x), L.dtype_code(x.dtype), 1, R, C, ptr(ones), ptr(out), ptr(ws), ws_bytes,
         stream_ptr(x.device))
    return out


class _TokenRouter(torch.autograd.Function):
    """The per-token router in one function: logits = x W^T + b (router.py:294, fp32 logits from
    bf16 operands) and the top-k chain (router.py:114-149 over every token).  Returns (logits,
    idx, w); the logits are an output for the router losses.  Backward: moc_router_topk_bwd_pack
    turns dw (plus the logits' own gradient, when the losses took one) straight into the bf16
    operand of the two products and the bias gradient, so the fp32 logit gradient is never
    written; then dx on the rows GEMM (zero-padded W^T) and dW on the split-row weight gradient,
    as _TokenRouterLinear does from a materialised logit gradient."""

    @staticmethod
    def forward(ctx, x, W, b, k, S):
        Wc = W.to(x.dtype).contiguous()
        R, K = x.shape
        C = Wc.shape[0]
        dev = x.device
        logits = torch.empty(R, C, device=dev, dtype=torch.float32)
        bias = None if b is None else b.float().contiguous()
        st = stream_ptr(dev)
        call("moc_rows_linear_f32", ptr(x), K, R, ptr(Wc), C, K, None if bias is None else ptr(bias), ptr(logits), C, st)
        idx = torch.empty(R, k, device=dev, dtype=torch.int32)
        w = torch.empty(R, k, device=dev, dtype=torch.float32)
        call("moc_router_topk", ptr(logits), R, C, S, k, ptr(idx), ptr(w), None, st)
        ctx.save_for_backward(x, Wc, logits, idx)
        ctx.meta = (W.dtype, None if b is None else b.dtype, int(k), int(S))
        ctx.mark_non_differentiable(idx)
        ctx.set_materialize_grads(False)
        return logits, idx, w

    @staticmethod
    def backward(ctx, dlogits, _didx, dw):
        x, Wc, logits, idx = ctx.saved_tensors
        w_dtype, b_dtype, k, S = ctx.meta
        if dw is None and dlogits is None:
            return None, None, None, None, None
        R, K = x.shape
        C = Wc.shape[0]
        dev = x.device
        st = stream_ptr(dev)
        dwc = torch.zeros(R, k, device=dev, dtype=torch.float32) if dw is None else dw.float().contiguous()
        dzin = None if dlogits is None else dlogits.float().contiguous()
        Cp = (C + 255) // 256 * 256
        dzp = torch.empty(R, Cp, device=dev, dtype=torch.bfloat16)
        db32 = torch.empty(C, device=dev, dtype=torch.float32)
        ws_bytes = L.query("moc_router_topk_bwd_pack_workspace", R, C)
        ws = torch.empty(max(1, ws_bytes // 4), device=dev, dtype=torch.float32)
        call("moc_router_topk_bwd_pack", ptr(logits), ptr(idx), ptr(dwc), R, C, S, k, ptr(dzin), Cp, ptr(dzp),
             ptr(db32), ptr(ws), ws_bytes, st)
        dx = dW = db = None
        if ctx.needs_input_grad[0]:
            wt = torch.empty(K, Cp, device=dev, dtype=torch.bfloat16)
            call("moc_weight_transpose", ptr(Wc), L.dtype_code(Wc.dtype), C, K, ptr(wt), Cp, st)
            dx = rows_linear(dzp, wt)
        if ctx.needs_input_grad[1]:
            dW = linear_wgrad(dzp, x, torch.float32)[:C].to(w_dtype)
        if ctx.needs_input_grad[2] and b_dtype is not None:
            db = db32.to(b_dtype)
        return dx, dW, db, None, None


def token_router_fused_ok(x: torch.Tensor, C: int, k: int) -> bool:
    """Whether _TokenRouter takes these rows (bf16 tokens, d % 256 == 0, the one-wave-per-row
    top-k kernels: more than 64 rows, C <= 4,608, k <= 64)."""
    R, K = x.shape
    return x.dtype == torch.bfloat16 and K % 256 == 0 and R > 64 and C <= 4608 and 0 < k <= 64


def token_router(h: torch.Tensor, W: torch.Tensor, b: Optional[torch.Tensor], k: int, S: int):
    """(logits (B*T, C) fp32, idx int32 (B*T, k), w fp32 (B*T, k)) of the per-token router
    (router.py:262-340): fused when token_router_fused_ok, else the logits GEMM and the top-k
    chain as two functions."""
    L.require_gpu(h, W)
    x = h.reshape(-1, h.shape[-1])
    if token_router_fused_ok(x, W.shape[0], k):
        return _TokenRouter.apply(x.contiguous(), W, b, int(k), int(S))
    logits = router_token_logits(h, W, b)
    idx, w = router_topk(logits, k, S)
    return logits, idx, w


def router_token_logits(h: torch.Tensor, W: torch.Tensor, b: Optional[torch.Tensor]) -> torch.Tensor:
    """Per-token router logits (B*T, C) in fp32 (router.py:294); see _TokenRouterLinear."""
    L.require_gpu(h, W)
    x = h.reshape(-1, h.shape[-1])
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.float()
    return _TokenRouterLinear.apply(x.contiguous(), W, b)


def token_routed_attention(q, routed_memory, wk, wv, idx, chapter_weights, *, tokens_per_chapter: int,
                           version: str = "v2", num_kv_heads: Optional[int] = None):
    """Routed branch of the token-level memory layer (see memory_amd.sparse_attention)."""
    from .sparse_attention import token_routed_attention as _tra
    return _tra(q, routed_memory, wk, wv, idx, chapter_weights, tokens_per_chapter=tokens_per_chapter,
                version=version, num_kv_heads=num_kv_heads)
