"""The sequence-routed memory layer as one autograd function with a stream-scheduled backward.

Reference chain (one memory layer of MemoryTransformer.forward, memory_transformer/model.py:609-692,
and the sublayer call memory_block.py:549-558 without the caller-owned norm and residual):
mean-pool -> router linear -> softmax / top-k (router.py:96-149) -> shared-chapter prepend
(model.py:356-391) -> gather x omega -> k_proj / v_proj -> attention -> o_proj
(memory_attention.py:241-243, :269-478).

The same kernels as the per-op autograd functions of ``ops``, scheduled as one unit:

forward    main stream: pool -> router linear -> top-k + prepend (one launch) -> chapter plan ->
           K/V projection -> attention -> o_proj;
           aux stream, beside the router chain (which is latency-bound: a few workgroups per
           launch): the q projection and the [Wk; Wv] pack, which do not depend on the routing.
backward   main stream: o_proj dX -> attention backward (dQ, then dK/dV) -> K/V weight gradient ->
           dX of the projection into the bank rows;
           aux stream: o_proj dW beside the o_proj dX and the dQ kernel; after dQ the q projection's
           dX and dW beside the dK/dV kernel; after dK/dV the router's backward (d omega partials ->
           dlogits -> router linear backward) and the pooling's gradient added into dh, beside
           the K/V chapter GEMMs.  The main stream waits for the aux stream before returning.

Every tensor the aux stream writes and the caller sees is allocated on the main stream before
the fork, so the caching allocator never hands its memory to another stream early.

For a plain bf16 bank (no row norm, no BankAdamW mirror, no row-sparse gradient) the same schedule
runs natively: moc_seq_layer_fwd / moc_seq_layer_bwd issue every launch, event and stream wait
from C++ (the q / o projections on the chapter GEMM, their transposed weights packed in the
forward), so a training step costs two host calls; PyTorch only allocates the outputs, one saved
buffer and one scratch buffer.  ``NATIVE = False`` keeps the Python-scheduled sequence.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from . import _lib as L
from . import ops
from ._lib import call, ptr, stream_ptr


def supported(h: torch.Tensor, bank: torch.Tensor, wq: torch.Tensor, wo: torch.Tensor, wr: torch.Tensor,
              num_shared: int, top_k: int, num_chapters: int, T: int) -> bool:
    """Whether the fused layer handles this configuration (otherwise the per-op path runs)."""
    d = h.shape[-1]
    return (h.is_cuda and h.dim() == 3 and h.dtype == torch.bfloat16 and wq.dtype == torch.bfloat16
            and wo.dtype == torch.bfloat16 and wr.dtype in (torch.float32, torch.bfloat16) and d % 8 == 0
            and 0 < num_shared <= 1024 and 0 < top_k <= 1024 and top_k <= num_chapters - num_shared
            and num_chapters <= 8192 and h.shape[0] <= 64 and T == 64 and h.shape[1] > 0)


NATIVE = True


def _native_saved_bytes(h, bank, wr, br, wq, wk, wv, wo, cfg) -> int:
    """Bytes of the native path's saved buffer, or 0 when the layer's configuration is outside
    moc_seq_layer_fwd / _bwd (those then run as the Python-scheduled sequence below)."""
    if not NATIVE:
        return 0
    C, T, S, k, scale, H, HK, norm, eps = cfg
    B, Lq, d = h.shape
    if (norm != L.MOC_NORM_NONE or bank.dtype != torch.bfloat16 or bank.dim() != 2 or bank.shape[1] != d
            or T != 64 or d != 64 * H or any(t.dtype != torch.bfloat16 for t in (wq, wk, wv, wo))
            or getattr(bank, "_moc_bank_opt", None) is not None or getattr(bank, "_moc_row_grad", None) is not None
            or (br is not None and br.dtype not in (torch.float32, torch.bfloat16))):
        return 0
    return int(L.query("moc_seq_layer_saved_bytes", B, Lq, d, H, HK, C, S, k))


class _SeqRoutedLayer(torch.autograd.Function):
    @staticmethod
    def forward(ctx, h, bank, wr, br, wq, wk, wv, wo, coef, cfg):
        C, T, S, k, scale, H, HK, norm, eps = cfg
        dev = h.device
        B, Lq, d = h.shape
        Dh = d // H
        KV = HK * Dh
        NS = S + k
        h = h.contiguous()
        ctx.cfg = cfg
        ctx.wdt = (wr.dtype, None if br is None else br.dtype)
        ctx.set_materialize_grads(False)
        nbytes = _native_saved_bytes(h, bank, wr, br, wq, wk, wv, wo, cfg)
        ctx.native = nbytes > 0
        if ctx.native:
            # the whole forward in one host call (moc_seq_layer_fwd)
            main = torch.cuda.current_stream(dev)
            aux = ops._side_stream(dev, "aux")
            wrc = wr.contiguous()
            brc = None if br is None else br.float().contiguous()
            cf = None if coef is None else coef.to(device=dev, dtype=torch.float32).contiguous()
            saved = torch.empty(nbytes, device=dev, dtype=torch.uint8)
            out = torch.empty(B, Lq, d, device=dev, dtype=h.dtype)
            logits = torch.empty(B, C, device=dev, dtype=torch.float32)
            idx = torch.empty(B, k, device=dev, dtype=torch.int32)
            idx_star = torch.empty(B, NS, device=dev, dtype=torch.int32)
            omega = torch.empty(B, NS, device=dev, dtype=torch.float32)
            wq, wk, wv, wo, bank = wq.contiguous(), wk.contiguous(), wv.contiguous(), wo.contiguous(), bank.contiguous()
            call("moc_seq_layer_fwd", ptr(h), ptr(bank), ptr(wrc), L.dtype_code(wrc.dtype), ptr(brc), ptr(wq),
                 ptr(wk), ptr(wv), ptr(wo), ptr(cf), B, Lq, d, H, HK, C, S, k, float(scale), ptr(out), ptr(logits),
                 ptr(idx), ptr(idx_star), ptr(omega), ptr(saved), nbytes, main.cuda_stream, aux.cuda_stream)
            ctx.save_for_backward(h, bank, wrc, cf, logits, idx, omega, saved)
            ctx.mark_non_differentiable(idx, idx_star, omega)
            return out, logits, idx, idx_star, omega
        h2 = h.view(B * Lq, d)
        main = torch.cuda.current_stream(dev)
        aux = ops._side_stream(dev, "aux")

        # aux: q projection and the K/V weight pack (outputs allocated on the main stream)
        q = torch.empty(B * Lq, d, device=dev, dtype=h.dtype)
        wkv = torch.empty(2 * KV, d, device=dev, dtype=torch.bfloat16)
        wqc, wkc, wvc = wq.contiguous(), wk.contiguous(), wv.contiguous()
        aux.wait_stream(main)
        with torch.cuda.stream(aux):
            with L.region("lib_linear_fwd"):
                torch.matmul(h2, wqc.t(), out=q)
            call("moc_weight_pack", ptr(wkc), L.dtype_code(wkc.dtype), ptr(wvc), L.dtype_code(wvc.dtype), KV, d,
                 ptr(wkv), None, aux.cuda_stream)
        q_ready = torch.cuda.Event()
        q_ready.record(aux)

        # main: router (pool -> linear -> top-k + prepend)
        st = main.cuda_stream
        cf = None if coef is None else coef.to(device=dev, dtype=torch.float32).contiguous()
        pooled = torch.empty(B, d, device=dev, dtype=torch.float32)
        call("moc_router_pool1", ptr(h), L.dtype_code(h.dtype), B, Lq, d, ptr(cf), ptr(pooled), st)
        wrc = wr.contiguous()
        brc = None if br is None else br.float().contiguous()
        logits = torch.empty(B, C, device=dev, dtype=torch.float32)
        call("moc_router_linear", ptr(pooled), B, d, ptr(wrc), L.dtype_code(wrc.dtype), ptr(brc), C, ptr(logits), st)
        idx = torch.empty(B, k, device=dev, dtype=torch.int32)
        w = torch.empty(B, k, device=dev, dtype=torch.float32)
        idx_star = torch.empty(B, NS, device=dev, dtype=torch.int32)
        omega = torch.empty(B, NS, device=dev, dtype=torch.float32)
        call("moc_router_topk_prepend", ptr(logits), B, C, S, k, float(scale), ptr(idx), ptr(w), ptr(idx_star),
             ptr(omega), st)

        # main: plan, K/V projection, attention (waits for q and the packed weights)
        main.wait_event(q_ready)
        out_attn, saved, acfg = ops.routed_attn_forward(q.view(B, Lq, H, Dh), bank, wk, wv, omega, idx_star, C, T,
                                                        norm, eps, HK, wkv=wkv)
        a2 = out_attn.view(B * Lq, d)
        with L.region("lib_linear_fwd"):
            out = F.linear(a2, wo)
        ctx.row_grad = getattr(bank, "_moc_row_grad", None)
        ctx.save_for_backward(h, wrc, wqc, wo, pooled, logits, idx, w, cf, *saved)
        ctx.acfg = acfg
        ctx.mark_non_differentiable(idx, idx_star, omega)
        return out.view(B, Lq, d), logits, idx, idx_star, omega

    @staticmethod
    def backward(ctx, dout, dlogits, _didx, _didx_star, _domega):
        if ctx.native:
            return _native_backward(ctx, dout, dlogits)
        h, wrc, wqc, wo, pooled, logits, idx, w, cf = ctx.saved_tensors[:9]
        saved = ctx.saved_tensors[9:]
        C, T, S, k, scale, H, HK, norm, eps = ctx.cfg
        need_h, need_bank, need_wr, need_br, need_wq, need_wk, need_wv, need_wo = ctx.needs_input_grad[:8]
        dev = h.device
        B, Lq, d = h.shape
        Dh = d // H
        a2 = saved[4].view(B * Lq, d)          # attention output (the o_proj input)
        main = torch.cuda.current_stream(dev)
        aux = ops._side_stream(dev, "aux")
        dh = dwr = dbr = dwq = dwo = None
        if dout is None:
            dout = torch.zeros(B, Lq, d, device=dev, dtype=h.dtype)
        dout2 = dout.reshape(B * Lq, d).to(h.dtype).contiguous()

        # aux: o_proj dW beside the o_proj dX and the attention backward's first kernels
        if need_wo:
            dwo = torch.empty(wo.shape, device=dev, dtype=wo.dtype)
            aux.wait_stream(main)
            with torch.cuda.stream(aux):
                ops.linear_wgrad(dout2, a2, wo.dtype, out=dwo)
        with L.region("lib_linear_dx"):
            d_attn = torch.matmul(dout2, wo)
        if need_h:
            dh = torch.empty(B, Lq, d, device=dev, dtype=h.dtype)
        if need_wq:
            dwq = torch.empty(wqc.shape, device=dev, dtype=wqc.dtype)

        def after_dq(dq):
            # aux: the q projection's dX (into dh) and dW beside the dK/dV kernel
            if not (need_h or need_wq):
                return
            aux.wait_stream(main)
            with torch.cuda.stream(aux):
                dq2 = dq.view(B * Lq, d)
                if need_h:
                    with L.region("lib_linear_dx"):
                        torch.matmul(dq2, wqc, out=dh.view(B * Lq, d))
                if need_wq:
                    ops.linear_wgrad(dq2, h.view(B * Lq, d), wqc.dtype, out=dwq)

        router_out = {}

        def after_dkv(dom_part):
            # aux: the router's backward and the pooling's gradient, beside the K/V chapter GEMMs
            if not (need_h or need_wr or need_br):
                return
            dz = torch.empty(B, C, device=dev, dtype=torch.float32)
            dpooled = torch.empty(B, d, device=dev, dtype=torch.float32) if need_h else None
            dW = torch.empty(C, d, device=dev, dtype=torch.float32) if need_wr else None
            db = torch.empty(C, device=dev, dtype=torch.float32) if need_br else None
            ws = None
            if dpooled is not None:
                ws = torch.empty(L.query("moc_router_linear_bwd_workspace", B, d, C) // 4, device=dev,
                                 dtype=torch.float32)
            dz_in = None if dlogits is None else dlogits.float().contiguous()
            aux.wait_stream(main)
            sa = aux.cuda_stream
            call("moc_router_seq_bwd", ptr(logits), ptr(idx), ptr(w), ptr(dom_part), HK, B, C, S, k, float(scale),
                 ptr(dz_in), ptr(dz), sa)
            call("moc_router_linear_bwd", ptr(dz), ptr(pooled), B, d, ptr(wrc), L.dtype_code(wrc.dtype), C,
                 ptr(dpooled), ptr(dW), ptr(db), ptr(ws), 0 if ws is None else ws.numel() * 4, sa)
            if dpooled is not None:
                call("moc_rows_add_bcast", ptr(dh), L.dtype_code(dh.dtype), B, Lq, d, ptr(dpooled), ptr(cf),
                     1.0 / Lq, sa)
            # kept alive (and unused by the main stream) until the main stream has waited for aux
            router_out.update(dz=dz, dpooled=dpooled, ws=ws, dz_in=dz_in, dom_part=dom_part, dW=dW, db=db)

        dq, dbank, dwk, dwv, _ = ops.routed_attn_backward(
            saved, ctx.acfg, d_attn.view(B, Lq, H, Dh), (True, need_bank, need_wk, need_wv, True),
            row_grad=ctx.row_grad, after_dq=after_dq, after_dkv=after_dkv)
        main.wait_stream(aux)
        if need_wr:
            dwr = router_out["dW"].to(ctx.wdt[0])
        if need_br:
            dbr = router_out["db"].to(ctx.wdt[1])
        return dh, dbank, dwr, dbr, dwq, dwk, dwv, dwo, None, None


def _native_backward(ctx, dout, dlogits):
    """The whole backward in one host call (moc_seq_layer_bwd)."""
    h, bank, wrc, cf, logits, idx, omega, saved = ctx.saved_tensors
    C, T, S, k, scale, H, HK, norm, eps = ctx.cfg
    need_h, need_bank, need_wr, need_br, need_wq, need_wk, need_wv, need_wo = ctx.needs_input_grad[:8]
    dev = h.device
    B, Lq, d = h.shape
    KV = HK * 64
    if dout is None:
        dout = torch.zeros(B, Lq, d, device=dev, dtype=h.dtype)
    dout = dout.to(h.dtype).contiguous()
    dz_in = None if dlogits is None else dlogits.float().contiguous()
    dh = torch.empty(B, Lq, d, device=dev, dtype=h.dtype) if need_h else None
    dbank = torch.empty(bank.shape, device=dev, dtype=bank.dtype) if need_bank else None
    dwr = torch.empty(C, d, device=dev, dtype=torch.float32) if need_wr else None
    dbr = torch.empty(C, device=dev, dtype=torch.float32) if need_br else None
    dwq = torch.empty(d, d, device=dev, dtype=torch.bfloat16) if need_wq else None
    dwkv = torch.empty(2 * KV, d, device=dev, dtype=torch.bfloat16) if (need_wk or need_wv) else None
    dwo = torch.empty(d, d, device=dev, dtype=torch.bfloat16) if need_wo else None
    nscratch = int(L.query("moc_seq_layer_scratch_bytes", B, Lq, d, H, HK, C, S, k))
    scratch = torch.empty(nscratch, device=dev, dtype=torch.uint8)
    main = torch.cuda.current_stream(dev)
    aux = ops._side_stream(dev, "aux")
    fill = ops._side_stream(dev, "fill")
    call("moc_seq_layer_bwd", ptr(h), ptr(bank), ptr(wrc), L.dtype_code(wrc.dtype), ptr(cf), B, Lq, d, H, HK, C, S, k,
         float(scale), ptr(logits), ptr(idx), ptr(omega), ptr(saved), saved.numel(), ptr(dout), ptr(dz_in), ptr(dh),
         ptr(dbank), bank.shape[0], ptr(dwr), ptr(dbr), ptr(dwq), ptr(dwkv), L.MOC_BF16, ptr(dwo), ptr(scratch),
         nscratch, main.cuda_stream, aux.cuda_stream, fill.cuda_stream)
    dwk = dwkv[:KV] if need_wk else None
    dwv = dwkv[KV:] if need_wv else None
    if dwr is not None:
        dwr = dwr.to(ctx.wdt[0])
    if dbr is not None:
        dbr = dbr.to(ctx.wdt[1])
    return dh, dbank, dwr, dbr, dwq, dwk, dwv, dwo, None, None


def seq_routed_layer(h, bank, wr, br, wq, wk, wv, wo, *, num_chapters: int, tokens_per_chapter: int,
                     num_shared: int, top_k: int, routed_scale: float, num_heads: int, num_kv_heads: int,
                     norm_type: Optional[str] = None, eps: float = 1e-6, coef: Optional[torch.Tensor] = None):
    """(out (B, L, d), logits f32 (B, C), idx int32 (B, k), idx_star int32 (B, S+k), omega f32 (B, S+k))."""
    cfg = (int(num_chapters), int(tokens_per_chapter), int(num_shared), int(top_k), float(routed_scale),
           int(num_heads), int(num_kv_heads), ops.norm_code(norm_type), float(eps))
    return _SeqRoutedLayer.apply(h, bank, wr, br, wq, wk, wv, wo, coef, cfg)
