"""Token-routed sparse memory attention on libmoc's chapter-centric kernels.

Entry points with the reference's signatures:
  * FSA_topk_sparse_attention_bthd            (kernels-final/kernel_v2.py:3181-3195; v1-v3)
  * FSA_topk_sparse_attention_weighted_bthd   (kernels-final/kernel_v4.py:1313-1326; v4)
  * FSA_topk_sparse_attention_weighted_joint_bias_bthd
                                              (kernels-final/kernel_v5.py:819; v5, same signature)
and ``token_routed_attention`` for MemoryCrossAttention's token path
(memory_attention.py:480-716), which projects the routed bank once per call
instead of once per batch element.

Combine modes (see csrc/sparse_xattn.hip): 0 = exact per-chapter MoE
(sum_s w_s softmax_s V_s); 1 = joint softmax over all selected keys;
2 = joint softmax with block weights p ~ max(w, 0) e^s (v1-v3 block_weights_bths);
3 = joint softmax with a log(max(w, 1e-20)) logit bias (v5).
The kernels work on 64-key blocks (head_dim 64); block sizes that are multiples of 64 are taken
as consecutive 64-key blocks (the per-chapter MoE combine then one joint call per slot); fp32,
bf16, and fp16 through the fp32 kernels.  Packed variable-length inputs (cu_seqlens_q /
cu_seqlens_k) run as one batch row with global block ids when every sequence's keys start and
end on a 64-key boundary.
"""

from __future__ import annotations

from typing import List, Optional

import torch
import torch.nn.functional as F

from . import _lib as L
from ._lib import call, ptr, stream_ptr
from . import ops

BLOCK = 64


class _Segment:
    """One plan over the edges of a set of kv heads (all heads when the chapter
    choice is the same for every head, else one kv head)."""

    def __init__(self, chap_flat: torch.Tensor, num_chapters: int, hk0: int, nhk: int, hq_off: int, rpe: int,
                 w_flat: Optional[torch.Tensor]):
        self.plan = ops.chapter_plan(chap_flat, num_chapters)
        self.hk0, self.nhk, self.hq_off, self.rpe = hk0, nhk, hq_off, rpe
        self.w = w_flat
        self.E = chap_flat.numel()


def _kv_strides(layout: str, HK: int):
    """Element strides (chapter, kv head, row) of a K/V buffer."""
    if layout == "natural":   # [chapters*64][HK][64]
        return 64 * HK * 64, 64, HK * 64
    if layout == "tiles":     # [chapters][HK][64][64]
        return HK * 64 * 64, 64 * 64, 64
    raise ValueError(layout)


def _kv_geom(layout: str, k: torch.Tensor):
    """(HK, (chapter, kv head, row) element strides) of a K or V operand.  "rows" is a
    [chapters*64, HK*64] view with any row stride (K or V columns of a fused KV GEMM output)."""
    if layout == "natural":
        HK = k.shape[-2]
    elif layout == "tiles":
        HK = k.shape[1]
    elif layout == "rows":
        rs = k.stride(0)
        return k.shape[1] // 64, (64 * rs, 64, rs)
    else:
        raise ValueError(layout)
    return HK, _kv_strides(layout, HK)


def _forward(q, k, v, layout, segments: List[_Segment], mode: int, S: int, scale: float):
    B, Tq, HQ, D = q.shape
    HK, (cs, hs, rs) = _kv_geom(layout, k)
    dt = L.dtype_code(q.dtype)
    st = stream_ptr(q.device)
    ntok = B * Tq
    out = torch.empty(B, Tq, HQ, D, device=q.device, dtype=q.dtype)
    saved = []
    for sg in segments:
        o_part = torch.empty(sg.E * sg.rpe, D, device=q.device, dtype=q.dtype)   # partials in the data dtype
        lse_part = torch.empty(sg.E * sg.rpe, device=q.device, dtype=torch.float32)
        call("moc_sparse_fwd", dt, ptr(q), ntok, HQ, ptr(k), ptr(v), cs, hs, rs, HK, D, ptr(sg.plan.uniq),
             ptr(sg.plan.n_uniq), ptr(sg.plan.csr_off), ptr(sg.plan.csr_edge), sg.plan.max_u, S, sg.hk0, sg.nhk,
             sg.hq_off, sg.rpe, float(scale), ptr(o_part), ptr(lse_part), st)
        lse_joint = None if mode == 0 else torch.empty(ntok * sg.rpe, device=q.device, dtype=torch.float32)
        call("moc_sparse_combine", dt, ptr(o_part), ptr(lse_part), ptr(sg.plan.edge_u), ptr(sg.w), mode, S, sg.rpe,
             ntok, HQ, sg.hq_off, ptr(out), ptr(lse_joint), st)
        # the backward needs the per-edge lse (mode 0) or the joint lse (modes 1-3), not o_part
        saved.append((lse_part if mode == 0 else None, lse_joint))
        del o_part
    return out, saved


def _backward(q, k, v, layout, out, dout, segments, saved, mode, S, scale, dk, dv, dk_layout,
              zero_chapters: int = 0):
    """Fills dk/dv (layout dk_layout), returns dq and the per-edge dw (or None).  dk/dv are
    pre-zeroed, or, with zero_chapters = C > 0, uninitialised: the blocks of the C chapters
    that a segment's plan does not touch are zeroed here (the touched ones are written whole)."""
    B, Tq, HQ, D = q.shape
    HK, (cs, hs, rs) = _kv_geom(layout, k)
    dt = L.dtype_code(q.dtype)
    st = stream_ptr(q.device)
    ntok = B * Tq
    dq = torch.empty_like(q)
    dws = []
    dout = dout.to(q.dtype).contiguous()
    ocs, ohs, ors, dv_off = dk_layout
    for sg, (lse_part, lse_joint) in zip(segments, saved):
        if mode == 0:
            # per-chapter deltas dO . o_s, written by moc_sparse_bwd itself
            drow = torch.empty(sg.E * sg.rpe, device=q.device, dtype=torch.float32)
            lrow = lse_part
        else:
            drow = torch.empty(ntok * sg.rpe, device=q.device, dtype=torch.float32)
            lrow = lse_joint
            call("moc_sparse_bwd_prep", dt, ptr(dout), ptr(out), None, ptr(sg.plan.edge_u), mode, S, sg.rpe,
                 ntok, HQ, sg.hq_off, ptr(drow), st)
        dv_ptr = dv.data_ptr() if dv is not None else dk.data_ptr() + dv_off
        if zero_chapters:
            mark = torch.empty(zero_chapters, device=q.device, dtype=torch.int32)
            call("moc_sparse_zero_untouched", dt, ptr(dk), dv_ptr, ocs, ohs, ors, zero_chapters, sg.hk0, sg.nhk,
                 ptr(sg.plan.uniq), ptr(sg.plan.n_uniq), sg.plan.max_u, ptr(mark), st)
        dq_part = torch.empty(sg.E * sg.rpe, D, device=q.device, dtype=q.dtype)
        dlog = torch.empty(sg.E * sg.rpe, device=q.device, dtype=torch.float32) if mode in (2, 3) else None
        row_tab = None
        if q.dtype == torch.bfloat16:
            # the first 32 edges of every distinct chapter: a unit's first row block is requested
            # together with its plan entries
            row_tab = torch.empty(sg.plan.max_u * 32, device=q.device, dtype=torch.int32)
            call("moc_plan_row_table", ptr(sg.plan.n_uniq), ptr(sg.plan.csr_off), ptr(sg.plan.csr_edge),
                 sg.plan.max_u, 32, ptr(row_tab), st)
        call("moc_sparse_bwd", dt, ptr(q), ptr(dout), ntok, HQ, ptr(k), ptr(v), cs, hs, rs, HK, D,
             ptr(sg.plan.uniq), ptr(sg.plan.n_uniq), ptr(sg.plan.csr_off), ptr(sg.plan.csr_edge), sg.plan.max_u, S,
             sg.hk0, sg.nhk, sg.hq_off, sg.rpe, mode, ptr(lrow), ptr(drow), ptr(sg.w), float(scale), ptr(dk),
             dv_ptr, ocs, ohs, ors, ptr(dq_part), ptr(dlog), ptr(row_tab), st)
        call("moc_sparse_dq_combine", dt, ptr(dq_part), ptr(sg.plan.edge_u), S, sg.rpe, ntok, HQ, sg.hq_off, ptr(dq),
             st)
        if mode != 1:
            dw = torch.empty(sg.E, device=q.device, dtype=torch.float32)
            call("moc_sparse_dw", ptr(drow if mode == 0 else dlog), ptr(sg.w), ptr(sg.plan.edge_u), mode, sg.rpe,
                 sg.E, ptr(dw), st)
            dws.append(dw)
    return dq, dws


def _global_chapters(idx: torch.Tensor, M: int, per_batch: bool) -> torch.Tensor:
    """Chapter ids in the plan's id space: b * M + c for per-batch K/V; -1 when c is out of range.
    int32 ids of a shared K/V pass through: the plan itself drops ids outside [0, M)."""
    if idx.dtype == torch.int32 and not per_batch:
        return idx
    bad = (idx < 0) | (idx >= M)     # on the caller's ids (64-bit ids are not wrapped first)
    c = idx.to(torch.int32)
    if per_batch:
        B = c.shape[0]
        shape = (B,) + (1,) * (c.dim() - 1)
        c = c + torch.arange(B, device=c.device, dtype=torch.int32).view(shape) * M
    return torch.where(bad, torch.full_like(c, -1), c)


def _segments(idx: torch.Tensor, w: Optional[torch.Tensor], mode: int, M: int, per_batch: bool, HQ: int, HK: int,
              num_chapters: int) -> List[_Segment]:
    """idx (B, T, S) -> one segment for all heads; (B, T, HK, S) -> one segment per kv head."""
    G = HQ // HK
    if idx.dim() == 3:
        chap = _global_chapters(idx, M, per_batch).contiguous()
        wf = None if w is None else w.float().contiguous()
        return [_Segment(chap.reshape(-1), num_chapters, 0, HK, 0, HQ, wf)]
    segs = []
    for hk in range(HK):
        chap = _global_chapters(idx[:, :, hk, :], M, per_batch).contiguous()
        if w is None:
            wf = None
        elif w.dim() == 4:
            wf = w[:, :, hk, :].float().contiguous()
        else:
            wf = w.float().contiguous()
        segs.append(_Segment(chap.reshape(-1), num_chapters, hk, 1, hk * G, G, wf))
    return segs


class _FSAFunction(torch.autograd.Function):
    """Sparse attention over per-batch K/V [B, Tk, HK, D] (the FSA entry points)."""

    @staticmethod
    def forward(ctx, q, k, v, w, idx, mode, scale):
        L.require_gpu(q, k, v, idx, w)
        B, Tq, HQ, D = q.shape
        Bk, Tk, HK, Dk = k.shape
        if D != 64 or Dk != 64:
            raise ValueError(f"head_dim must be 64 for the HIP kernels, got {D}/{Dk}")
        if Tk % BLOCK != 0:
            raise ValueError(f"Tk={Tk} must be a multiple of block_size {BLOCK}")
        if HQ % HK != 0:
            raise ValueError(f"HQ ({HQ}) must be a multiple of HK ({HK})")
        if Bk not in (1, B):
            raise ValueError(f"k/v batch {Bk} must be 1 or {B}")
        M = Tk // BLOCK
        q, k, v = q.contiguous(), k.to(q.dtype).contiguous(), v.to(q.dtype).contiguous()
        S = idx.shape[-1]
        segs = _segments(idx, w, mode, M, Bk > 1, HQ, HK, Bk * M)
        out, saved = _forward(q, k, v, "natural", segs, mode, S, scale)
        ctx.segs, ctx.saved_parts = segs, saved
        ctx.save_for_backward(q, k, v, out)
        ctx.mode, ctx.S, ctx.scale = mode, S, scale
        ctx.w_shape = None if w is None else w.shape
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out = ctx.saved_tensors
        HK = k.shape[2]
        dk = torch.zeros_like(k)
        dv = torch.zeros_like(v)
        cs, hs, rs = _kv_strides("natural", HK)
        dq, dws = _backward(q, k, v, "natural", out, dout, ctx.segs, ctx.saved_parts, ctx.mode, ctx.S, ctx.scale,
                            dk, dv, (cs, hs, rs, 0))
        dw = None
        if ctx.w_shape is not None and dws:
            if len(dws) == 1:
                dw = dws[0].view(ctx.w_shape)
            elif len(ctx.w_shape) == 4:      # per-head weights: one segment per kv head
                dw = torch.stack([x.view(ctx.w_shape[0], ctx.w_shape[1], ctx.w_shape[3]) for x in dws], dim=2)
            else:                            # per-token weights shared by every kv head
                dw = torch.stack(dws, 0).sum(0).view(ctx.w_shape)
        return dq, dk, dv, dw, None, None, None


def _check_common(cu_seqlens_q, cu_seqlens_k, disable_causal_mask, block_size):
    if (cu_seqlens_q is None) != (cu_seqlens_k is None):
        raise ValueError("cu_seqlens_q and cu_seqlens_k are given together")
    if not disable_causal_mask:
        raise NotImplementedError(
            "causal memory masking is not implemented; memory cross-attention is non-causal "
            "(MemoryCrossAttention passes disable_causal_mask=True, memory_attention.py:816)")
    bs = int(block_size)
    if bs < BLOCK or bs % BLOCK != 0:
        raise ValueError(f"block_size must be a multiple of {BLOCK} (the chapter tile of the HIP kernels), got "
                         f"{block_size}")


def _fsa(q, k, v, w, idx, mode: int, scale: float, block_size: int):
    """The FSA function over 64-key blocks.  A block of 64 m keys (joint modes) is m consecutive
    64-key blocks carrying the block's weight: the joint softmax over them is the joint softmax
    over the blocks, the block weight's gradient the sum of its sub-blocks' (autograd of the
    repeat), and a block reaching past the keys has its missing sub-blocks skipped as out of range
    (the reference masks those keys).  fp16 inputs run the fp32 kernels (exact widening), the
    output rounded back to fp16."""
    m = int(block_size) // BLOCK
    if m > 1:
        sub = torch.arange(m, device=idx.device, dtype=idx.dtype)
        idx = (idx.unsqueeze(-1) * m + sub).flatten(-2)    # negative ids stay negative
        if w is not None:
            w = w.repeat_interleave(m, dim=-1)
    half = q.dtype == torch.float16
    if half:
        q, k, v = q.float(), k.float(), v.float()
    out = _FSAFunction.apply(q, k, v, w, idx, mode, scale)
    return out.to(torch.float16) if half else out


def _varlen(q, k, v, idx, w, cu_q, cu_k, block_size):
    """Packed variable-length inputs (kernel_v2.py:3181-3330): the B * Tq query rows and B * Tk
    key rows hold sequences s = 0 .. n-1 at rows cu_q[s] .. cu_q[s+1] and cu_k[s] .. cu_k[s+1];
    a query's block b is keys b BS .. b BS + BS - 1 of its own sequence, blocks past the
    sequence skipped (a partial last block keeps the keys inside it).  When every sequence's
    keys start on a 64-key boundary and count a multiple of 64, block b of sequence s is the
    64-key blocks cu_k[s] / 64 + m b + j (j < m = BS / 64) of the packed keys that lie inside
    the sequence: the packed tensors run as one batch row with those ids (-1: skipped).
    Returns (q, k, v, ids (1, Nq, H, S m), weights repeated per sub-block or None)."""
    B, Tq = q.shape[0], q.shape[1]
    Nq, Nk = B * Tq, k.shape[0] * k.shape[1]
    cq = cu_q.detach().to("cpu", torch.int64)
    ck = cu_k.detach().to("cpu", torch.int64)
    if cq.dim() != 1 or ck.shape != cq.shape or cq.numel() < 2:
        raise ValueError("cu_seqlens_q / cu_seqlens_k must be 1-D of equal length n + 1")
    if int(cq[0]) != 0 or int(ck[0]) != 0 or int(cq[-1]) != Nq or int(ck[-1]) != Nk:
        raise ValueError(f"cu_seqlens must run from 0 to the packed lengths ({Nq} queries, {Nk} keys)")
    if bool((cq[1:] < cq[:-1]).any()) or bool((ck[1:] < ck[:-1]).any()):
        raise ValueError("cu_seqlens must be non-decreasing")
    if bool((ck % BLOCK != 0).any()):
        raise NotImplementedError(f"variable-length keys: every sequence's key rows must start and end on a "
                                  f"{BLOCK}-row boundary (the chapter tile of the HIP kernels)")
    m = int(block_size) // BLOCK
    dev = idx.device
    rows = torch.arange(Nq, device=dev)
    seq = torch.bucketize(rows, cq[1:].to(dev), right=True)
    kb0 = (ck.to(dev) // BLOCK)[seq]                                  # first 64-key block of the row's sequence
    nkb = ((ck[1:] - ck[:-1]).to(dev) // BLOCK)[seq]                  # its 64-key blocks
    ids = idx.reshape(Nq, idx.shape[2], idx.shape[3]).long()
    sub = (ids.unsqueeze(-1) * m + torch.arange(m, device=dev)).flatten(-2)
    ok = (ids.unsqueeze(-1) >= 0).expand(*ids.shape, m).flatten(-2) & (sub < nkb.view(Nq, 1, 1))
    gid = torch.where(ok, sub + kb0.view(Nq, 1, 1), torch.full_like(sub, -1)).to(torch.int32)
    if w is not None:
        w = w.reshape(1, Nq, *w.shape[2:]).repeat_interleave(m, dim=-1)
    return (q.reshape(1, Nq, *q.shape[2:]), k.reshape(1, Nk, *k.shape[2:]), v.reshape(1, Nk, *v.shape[2:]),
            gid.unsqueeze(0), w)


def _indices(block_indices_bths, topk_idx_hns, q):
    if block_indices_bths is not None:
        return block_indices_bths
    if topk_idx_hns is None:
        raise ValueError("block_indices_bths or topk_idx_hns is required")
    H, N, S = topk_idx_hns.shape
    B, Tq = q.shape[0], q.shape[1]
    return topk_idx_hns.permute(1, 0, 2).reshape(B, Tq, H, S)


def FSA_topk_sparse_attention_bthd(q_bthd, k_bthd, v_bthd, block_indices_bths, block_size, block_weights_bths=None,
                                   softmax_scale=None, cu_seqlens_q=None, cu_seqlens_k=None, topk_idx_hns=None,
                                   topk_w_hns=None, assume_sorted_topk=False, disable_causal_mask=False):
    """Joint softmax over each query's selected chapters (optionally block-weighted)."""
    _check_common(cu_seqlens_q, cu_seqlens_k, disable_causal_mask, block_size)
    idx = _indices(block_indices_bths, topk_idx_hns, q_bthd)
    w = block_weights_bths
    if w is None and topk_w_hns is not None:
        H, N, S = topk_w_hns.shape
        w = topk_w_hns.permute(1, 0, 2).reshape(q_bthd.shape[0], q_bthd.shape[1], H, S)
    scale = float(softmax_scale) if softmax_scale is not None else q_bthd.shape[-1] ** -0.5
    mode = 1 if w is None else 2
    if cu_seqlens_q is not None:
        q1, k1, v1, gid, w1 = _varlen(q_bthd, k_bthd, v_bthd, idx, w, cu_seqlens_q, cu_seqlens_k, block_size)
        return _fsa(q1, k1, v1, w1, gid, mode, scale, BLOCK).reshape(q_bthd.shape)
    return _fsa(q_bthd, k_bthd, v_bthd, w, idx, mode, scale, block_size)


def FSA_topk_sparse_attention_weighted_bthd(q_bthd, k_bthd, v_bthd, block_indices_bths, chapter_weights_bts,
                                            block_size, softmax_scale=None, cu_seqlens_q=None, cu_seqlens_k=None,
                                            topk_idx_hns=None, assume_sorted_topk=False, disable_causal_mask=False):
    """Exact per-chapter MoE combine: sum_s w_s softmax(q K_s^T) V_s (kernel_v4 semantics).  At
    block_size 64 m > 64 a block's softmax spans m 64-key blocks: each slot is then its own joint
    softmax over its m sub-blocks (one call per slot, the reference's per-chapter calls of
    memory_attention.py:640-707) and the slots are mixed by the weights."""
    _check_common(cu_seqlens_q, cu_seqlens_k, disable_causal_mask, block_size)
    idx = _indices(block_indices_bths, topk_idx_hns, q_bthd)
    scale = float(softmax_scale) if softmax_scale is not None else q_bthd.shape[-1] ** -0.5
    w = chapter_weights_bts
    m = int(block_size) // BLOCK
    if cu_seqlens_q is not None:
        q1, k1, v1, gid, _ = _varlen(q_bthd, k_bthd, v_bthd, idx, None, cu_seqlens_q, cu_seqlens_k, block_size)
        w1 = w.reshape(1, q1.shape[1], *w.shape[2:])
        if m == 1:
            return _fsa(q1, k1, v1, w1, gid, 0, scale, BLOCK).reshape(q_bthd.shape)
        out = None
        for sl in range(idx.shape[-1]):
            o = _fsa(q1, k1, v1, None, gid[..., sl * m:(sl + 1) * m], 1, scale, BLOCK)
            ws = w1[..., sl]
            ws = ws.unsqueeze(-1).unsqueeze(-1) if ws.dim() == 2 else ws.unsqueeze(-1)
            term = o.float() * ws.float()
            out = term if out is None else out + term
        return out.to(q_bthd.dtype).reshape(q_bthd.shape)
    if m == 1:
        return _fsa(q_bthd, k_bthd, v_bthd, w, idx, 0, scale, block_size)
    out = None
    for sl in range(idx.shape[-1]):
        o = _fsa(q_bthd, k_bthd, v_bthd, None, idx[..., sl:sl + 1], 1, scale, block_size)
        ws = w[..., sl]
        ws = ws.unsqueeze(-1).unsqueeze(-1) if ws.dim() == 2 else ws.unsqueeze(-1)   # (B, T[, H]) -> broadcast
        term = o.float() * ws.float()
        out = term if out is None else out + term
    return out.to(q_bthd.dtype)


def FSA_topk_sparse_attention_weighted_joint_bias_bthd(q_bthd, k_bthd, v_bthd, block_indices_bths,
                                                       chapter_weights_bts, block_size, softmax_scale=None,
                                                       cu_seqlens_q=None, cu_seqlens_k=None, topk_idx_hns=None,
                                                       assume_sorted_topk=False, disable_causal_mask=False):
    """Joint softmax with a log(max(w, 1e-20)) logit bias per chapter (kernel_v5 semantics)."""
    _check_common(cu_seqlens_q, cu_seqlens_k, disable_causal_mask, block_size)
    idx = _indices(block_indices_bths, topk_idx_hns, q_bthd)
    scale = float(softmax_scale) if softmax_scale is not None else q_bthd.shape[-1] ** -0.5
    if cu_seqlens_q is not None:
        q1, k1, v1, gid, w1 = _varlen(q_bthd, k_bthd, v_bthd, idx, chapter_weights_bts, cu_seqlens_q, cu_seqlens_k,
                                      block_size)
        return _fsa(q1, k1, v1, w1, gid, 3, scale, BLOCK).reshape(q_bthd.shape)
    return _fsa(q_bthd, k_bthd, v_bthd, chapter_weights_bts, idx, 3, scale, block_size)


# ------------------------------------------------------------------ model path

class _TokenRouted(torch.autograd.Function):
    """Routed branch of the token-level memory layer: K/V of the routed bank are
    projected once (one GEMM over every routed chapter), then sparse attention.

    q (B, L, H, 64); routed (N_r, d); wk/wv (HK*64, d); idx (B, L, k) local chapter
    ids; w (B, L, k) or None.  Returns (B, L, H, 64)."""

    @staticmethod
    def forward(ctx, q, routed, wk, wv, w, idx, mode, HK):
        L.require_gpu(q, routed, wk, wv, idx, w)
        dtype = q.dtype
        B, Lq, HQ, D = q.shape
        Nr, d = routed.shape
        if Nr % BLOCK != 0:
            raise ValueError(f"routed memory length {Nr} must be a multiple of {BLOCK}")
        C = Nr // BLOCK
        q = q.contiguous()
        routed = routed.contiguous()
        wkv_t = None
        if dtype == torch.bfloat16 and wk.shape[0] % 8 == 0 and wk.shape[1] % 8 == 0:
            # [Wk; Wv] and its transpose (the input gradient's operand) in one kernel
            wkv, wkv_t = ops.weight_pack(wk, wv, transposed=True)
        else:
            wkv = torch.cat([wk, wv], 0).to(dtype).contiguous()
        # every routed chapter is projected (no gather, no norm): one rows GEMM over the routed
        # bank (the chapter GEMM's wide tiles for bf16), K and V read by the sparse kernels as
        # strided column blocks of kv [Nr][2 KV]
        KV = HK * D
        rows = routed.to(dtype)
        if ops.rows_gemm_ok(rows, wkv):
            kv = ops.rows_linear(rows, wkv)
        else:
            with L.region("lib_token_kv_project"):
                kv = F.linear(rows, wkv)
        S = idx.shape[-1]
        segs = _segments(idx, w, mode, C, False, HQ, HK, C)
        out, saved = _forward(q, kv[:, :KV], kv[:, KV:], "rows", segs, mode, S, D ** -0.5)
        ctx.segs, ctx.saved_parts = segs, saved
        ctx.save_for_backward(q, routed, wkv, wkv_t, kv, out)
        ctx.cfg = (mode, S, HK, wk.dtype, wv.dtype, None if w is None else w.shape)
        return out

    @staticmethod
    def backward(ctx, dout):
        q, routed, wkv, wkv_t, kv, out = ctx.saved_tensors
        mode, S, HK, wk_dtype, wv_dtype, w_shape = ctx.cfg
        dtype = q.dtype
        D = q.shape[-1]
        KV = HK * D
        Nr, d = routed.shape
        # dk / dv written as rows [chapter*64 + key][hk*64 + dim] (dv at column offset KV); blocks
        # of chapters no token selected are zeroed by the backward instead of a 2 KV x Nr fill
        dkv = torch.empty(Nr, 2 * KV, device=q.device, dtype=dtype)
        elem = dkv.element_size()
        dq, dws = _backward(q, kv[:, :KV], kv[:, KV:], "rows", out, dout, ctx.segs, ctx.saved_parts, mode, S,
                            D ** -0.5, dkv, None, (64 * 2 * KV, 64, 2 * KV, KV * elem), zero_chapters=Nr // BLOCK)
        need_r, need_wk, need_wv = ctx.needs_input_grad[1:4]
        dr = dwk = dwv = None
        if need_wk or need_wv:
            dwkv = ops.linear_wgrad(dkv, routed, torch.float32 if torch.float32 in (wk_dtype, wv_dtype) else dtype)
            dwk = dwkv[:KV].to(wk_dtype) if need_wk else None
            dwv = dwkv[KV:].to(wv_dtype) if need_wv else None
        if need_r:
            dr = _rows_grad(routed, dkv, wkv, wkv_t)
        dw = None
        if w_shape is not None and dws:
            dw = dws[0].view(w_shape) if len(dws) == 1 else torch.stack(dws, 0).sum(0).view(w_shape)
        return dq, dr, dwk, dwv, dw, None, None, None


def _rows_grad(routed: torch.Tensor, dkv: torch.Tensor, wkv: torch.Tensor,
               wkv_t: Optional[torch.Tensor] = None) -> torch.Tensor:
    """d routed = dkv [Wk; Wv] (bf16: the chapter GEMM's rows mode with W = [Wk; Wv]^T).  When
    `routed` is the tail rows of a larger tensor (the routed part of a bank whose first rows are
    the shared chapters, split off by model.split_rows), the product is written into the tail of
    a buffer of the whole bank's shape, so the split's backward can hand that buffer on after
    filling the head rows instead of copying the tail."""
    if wkv_t is None:
        wkv_t = wkv.t().contiguous()
    native = ops.rows_gemm_ok(dkv, wkv_t)

    def product(out=None):
        if native:
            return ops.rows_linear(dkv, wkv_t, out=out)
        with L.region("lib_token_kv_dx"):
            return torch.mm(dkv, wkv, out=out) if out is not None else torch.matmul(dkv, wkv)

    base = routed._base
    if base is not None and base.dim() == 2 and base.is_contiguous() and routed.is_contiguous() \
            and base.shape[1] == routed.shape[1] and routed.dtype == dkv.dtype and base.dtype == routed.dtype:
        off = routed.storage_offset() - base.storage_offset()
        d = routed.shape[1]
        if off % d == 0 and off // d + routed.shape[0] == base.shape[0]:
            full = torch.empty(base.shape, device=dkv.device, dtype=dkv.dtype)
            full._moc_rows_tail = off // d        # read by model._SplitRows.backward
            tail = full[off // d:]
            product(tail)
            return tail
    return product().to(routed.dtype)


def token_routed_attention(q, routed_memory, wk, wv, idx, chapter_weights, *, tokens_per_chapter: int,
                           version: str = "v2", num_kv_heads: Optional[int] = None):
    """The routed branch of MemoryCrossAttention._forward_token_routed_attention
    (memory_attention.py:553-707), before routed_scale and o_proj.

    Dispatch mirrors the reference: weights given -> exact MoE combine (v1-v4),
    or the joint log-bias approximation when the version is v5; no weights ->
    joint softmax over the selected chapters."""
    T = int(tokens_per_chapter)
    if T <= 0 or T % BLOCK:
        raise ValueError(f"tokens_per_chapter must be a positive multiple of {BLOCK} for the HIP kernels, got {T}")
    HK = q.shape[2] if num_kv_heads is None else int(num_kv_heads)
    if chapter_weights is None:
        mode = 1
    else:
        mode = 3 if version == "v5" else 0
    w = None if chapter_weights is None else chapter_weights.float()
    m = T // BLOCK
    if m > 1:
        # the joint combines (no weights, v5's log-bias) see a chapter of 64 m rows as m
        # consecutive 64-row chapters with its weight; the per-chapter MoE combine would split
        # its softmax, so it keeps 64-row chapters
        if mode == 0:
            raise NotImplementedError(f"tokens_per_chapter {T}: the per-chapter MoE combine (kernel versions "
                                      "v1-v4 with chapter weights) needs 64-row chapters; v5 or no weights take "
                                      "any multiple of 64")
        sub = torch.arange(m, device=idx.device, dtype=torch.int64)
        idx = (idx.long().unsqueeze(-1) * m + sub).flatten(-2).to(idx.dtype)
        if w is not None:
            w = w.repeat_interleave(m, dim=-1)
    return _TokenRouted.apply(q, routed_memory, wk, wv, w, idx, mode, HK)
