"""PyTorch-CPU restatement of the reference MoC memory cross-attention path.

TEST INFRASTRUCTURE ONLY (see the package docstring): the checker for the HIP
path, never called by the product.

All functions take and return CPU tensors and compute in the dtype of their
inputs (tests use float64 for gradient pins and float32 for parity).
Citations are ``path:line`` inside the reference repository.

Tie rule for top-k (documented choice, see ``topk_desc``): values descending,
equal values ordered by ascending index.  ``torch.topk`` leaves tie order
unspecified, so this is the rule the HIP router implements and the oracle
restates.  Routing selects by *logit* (``select_by="logits"``), which is the
same set and order as selecting by the reference's masked, renormalised fp32
probabilities whenever distinct logits give distinct probabilities (softmax
and renormalisation are monotone); ``select_by="probs"`` restates the literal
probability chain for the pin of that equivalence.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F

__all__ = [
    "topk_desc", "topk_desc_numpy", "sequence_pool", "rolling_pool_coefficients",
    "linear", "route_sequence", "route_token_level", "router_losses",
    "compute_total_router_loss", "select_routed_chapters_from_probs",
    "prepend_shared_chapters", "normalize_shared_routed", "gather_chapters",
    "weight_memory", "compute_qkv", "attention", "cross_attention",
    "sequence_memory_layer", "token_routed_preproj", "token_memory_layer",
    "naive_reference_unweighted", "naive_reference_weighted",
    "naive_reference_weighted_joint_bias", "naive_reference_block_weighted",
    "sparse_attention_unweighted", "sparse_attention_weighted",
    "sparse_attention_joint_bias", "sparse_attention_block_weighted",
    "decode_step", "moe_with_routing", "rms_norm", "adamw_step", "clip_grad_norm",
    "block_rms_norm", "memory_sublayer", "masked_mean", "inference_route", "attention_weights",
]


# --------------------------------------------------------------------------
# top-k with the documented tie rule
# --------------------------------------------------------------------------

def topk_desc(x: torch.Tensor, k: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Top-k along the last dim, values descending, ties by ascending index.

    Restates ``torch.topk(x, k, dim=-1)`` (sorted=True) as used at
    memory_transformer/router.py:143, :322 and memory_transformer/model.py:352,
    with a fixed tie order (stable descending sort).
    """
    vals, idx = torch.sort(x, dim=-1, descending=True, stable=True)
    return vals[..., :k], idx[..., :k]


def topk_desc_numpy(x: np.ndarray, k: int) -> np.ndarray:
    """Brute-force index pin of ``topk_desc`` for 2-D arrays (lexsort)."""
    out = np.empty((x.shape[0], k), dtype=np.int64)
    for r in range(x.shape[0]):
        order = np.lexsort((np.arange(x.shape[1]), -x[r]))
        out[r] = order[:k]
    return out


# --------------------------------------------------------------------------
# router (memory_transformer/router.py)
# --------------------------------------------------------------------------

def rolling_pool_coefficients(L: int, window: Optional[int]) -> torch.Tensor:
    """c_l such that rolling-mean pooling == sum_l c_l * h_l.

    From router.py:158-195: pooled = mean_t mean(h[max(0,t-w+1):t+1]), so
    token l receives sum over t in [l, l+w-1] ∩ [0, L-1] of 1/(len_t * L),
    len_t = min(t+1, w).
    """
    w = L if window is None else int(window)
    if w <= 0:
        raise ValueError(f"rolling_window_size must be > 0, got {window}")
    w = min(w, L)
    c = torch.zeros(L, dtype=torch.float64)
    for t in range(L):
        ln = min(t + 1, w)
        c[max(0, t - w + 1): t + 1] += 1.0 / (ln * L)
    return c


def sequence_pool(h: torch.Tensor, strategy: str = "sequence",
                  window: Optional[int] = None) -> torch.Tensor:
    """Pooled router input: router.py:96-107 (mean) and :158-195 (rolling)."""
    if strategy == "sequence":
        return h.mean(dim=1)
    if strategy in ("sequence-rolling", "sequence_rolling"):
        B, L, D = h.shape
        w = L if window is None else int(window)
        if w <= 0:
            raise ValueError(f"rolling_window_size must be > 0, got {window}")
        w = min(w, L)
        cs = torch.cat([h.new_zeros((B, 1, D)), h.cumsum(dim=1)], dim=1)
        end = torch.arange(L) + 1
        start = torch.clamp(end - w, min=0)
        sums = cs[:, end, :] - cs[:, start, :]
        lens = (end - start).to(h.dtype).view(1, L, 1)
        return (sums / lens).mean(dim=1)
    raise ValueError(f"Unknown routing_strategy: {strategy}")


def linear(x: torch.Tensor, W: torch.Tensor, b: Optional[torch.Tensor] = None) -> torch.Tensor:
    """nn.Linear: x @ W^T + b."""
    y = x @ W.transpose(0, 1)
    return y if b is None else y + b


def _select(scores: torch.Tensor, logits: torch.Tensor, k: int, S: int,
            select_by: str) -> torch.Tensor:
    if select_by == "probs":
        return topk_desc(scores, k)[1]
    if select_by != "logits":
        raise ValueError(select_by)
    z = logits.clone()
    if S > 0:
        z[..., :S] = -math.inf
    return topk_desc(z, k)[1]


def route_sequence(logits: torch.Tensor, top_k: int, exclude_prefix_chapters: int = 0,
                   select_by: str = "logits"):
    """Sequence-level selection from router logits (router.py:114-149).

    Returns (indices int64 (R,k), weights (R,k), probs (R,C)).
    """
    R, C = logits.shape
    S = int(exclude_prefix_chapters)
    if S < 0 or S > C:
        raise ValueError(f"exclude_prefix_chapters must be in [0, {C}], got {S}")
    probs = F.softmax(logits, dim=-1)
    if S > 0:
        k = min(int(top_k), C - S)
        if k <= 0:
            return (torch.empty((R, 0), dtype=torch.long),
                    torch.empty((R, 0), dtype=probs.dtype), probs)
        p = probs.clone()
        p[:, :S] = 0.0
        p = p / p.sum(dim=-1, keepdim=True).clamp_min(1e-12)
        idx = _select(p, logits, k, S, select_by)
        w = torch.gather(p, -1, idx)
    else:
        k = int(top_k)
        idx = _select(probs, logits, k, 0, select_by)
        w = torch.gather(probs, -1, idx)
    w = w / w.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    return idx, w, probs


def route_token_level(logits: torch.Tensor, top_k: int, exclude_prefix_chapters: int = 0,
                      select_by: str = "logits"):
    """Token-level selection (router.py:262-340) from logits (B,T,C).

    Returns (global indices int64 (B,T,k), weights (B,T,k), probs (B,T,C)).
    """
    C = logits.shape[-1]
    S = int(exclude_prefix_chapters)
    if S < 0 or S > C:
        raise ValueError(f"exclude_prefix_chapters must be in [0, {C}], got {S}")
    probs = F.softmax(logits, dim=-1)
    k = min(int(top_k), C - S)
    if k <= 0:
        shp = logits.shape[:-1] + (0,)
        return torch.empty(shp, dtype=torch.long), torch.empty(shp, dtype=probs.dtype), probs
    routed = probs[..., S:]
    routed = routed / routed.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    if select_by == "probs":
        idx_local = topk_desc(routed, k)[1]
    else:
        idx_local = topk_desc(logits[..., S:], k)[1]
    w = torch.gather(routed, -1, idx_local)
    w = w / w.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    return idx_local + S, w, probs


def router_losses(logits: torch.Tensor, probs: torch.Tensor, idx: torch.Tensor,
                  num_chapters: int) -> Dict[str, torch.Tensor]:
    """Router auxiliary losses (router.py:197-260); rows are (R, C)."""
    C = int(num_chapters)
    one_hot = F.one_hot(idx, num_classes=C).to(probs.dtype)
    f = one_hot.sum(dim=1).mean(dim=0)
    P = probs.mean(dim=0)
    out = {"load_balance": C * (f * P).sum()}
    Psq = probs.pow(2).mean(dim=0)
    out["auxiliary"] = F.mse_loss(Psq, torch.ones_like(Psq) / C)
    lse = torch.logsumexp(logits, dim=-1)
    out["z_loss"] = (lse ** 2).mean()
    out["entropy"] = -(probs * torch.log(probs.clamp_min(1e-12))).sum(dim=-1).mean()
    return out


def compute_total_router_loss(losses, load_balance_coef=0.01, auxiliary_coef=0.0,
                              z_loss_coef=0.0):
    """router.py:490-527."""
    if not losses:
        return torch.tensor(0.0)
    total = next(iter(losses.values())).new_tensor(0.0)
    if "load_balance" in losses and load_balance_coef > 0:
        total = total + load_balance_coef * losses["load_balance"]
    if "auxiliary" in losses and auxiliary_coef > 0:
        total = total + auxiliary_coef * losses["auxiliary"]
    if "z_loss" in losses and z_loss_coef > 0:
        total = total + z_loss_coef * losses["z_loss"]
    return total


# --------------------------------------------------------------------------
# routing glue (memory_transformer/model.py)
# --------------------------------------------------------------------------

def select_routed_chapters_from_probs(probs: torch.Tensor, top_k: int, num_shared: int,
                                      select_by_scores: Optional[torch.Tensor] = None):
    """model.py:331-354.  Ties: ``topk_desc`` over ``select_by_scores`` (defaults
    to the masked probabilities themselves)."""
    R, C = probs.shape
    S = max(0, min(int(num_shared), C))
    k = min(int(top_k), C - S)
    if k <= 0:
        return torch.empty((R, 0), dtype=torch.long), torch.empty((R, 0), dtype=probs.dtype)
    p = probs.clone()
    if S > 0:
        p[:, :S] = 0.0
    p = p / p.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    if select_by_scores is None:
        idx = topk_desc(p, k)[1]
    else:
        z = select_by_scores.clone()
        if S > 0:
            z[:, :S] = -math.inf
        idx = topk_desc(z, k)[1]
    w = torch.gather(p, -1, idx)
    w = w / w.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    return idx, w


def prepend_shared_chapters(idx: torch.Tensor, w: torch.Tensor, *, num_chapters: int,
                            num_shared_chapters: int, routed_scaling_factor: float):
    """model.py:356-391: I* = [0..S-1, I], omega = [1.., s*w] / sum."""
    S = max(0, min(int(num_shared_chapters), int(num_chapters)))
    if S <= 0:
        return idx, w
    B = idx.shape[0]
    sidx = torch.arange(S, dtype=torch.long).unsqueeze(0).expand(B, -1)
    sw = torch.ones((B, S), dtype=w.dtype)
    if idx.shape[1] > 0:
        ci = torch.cat([sidx, idx], dim=-1)
        cw = torch.cat([sw, w * float(routed_scaling_factor)], dim=-1)
    else:
        ci, cw = sidx, sw
    cw = cw / cw.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    return ci, cw


def rms_norm(x: torch.Tensor, eps: float) -> torch.Tensor:
    """Row RMS normalisation without affine (model.py:423-425)."""
    return x / x.pow(2).mean(dim=-1, keepdim=True).add(eps).sqrt()


def normalize_shared_routed(memory: torch.Tensor, *, num_shared_chapters: int,
                            tokens_per_chapter: int, norm_type: str, eps: float):
    """model.py:393-432 (note: no-op unless both slices are non-empty)."""
    if memory.dim() != 3:
        raise ValueError(f"memory must be 3D (B, T, D), got shape {tuple(memory.shape)}")
    if tokens_per_chapter <= 0:
        return memory
    st = max(0, int(num_shared_chapters)) * int(tokens_per_chapter)
    st = min(st, int(memory.shape[1]))
    if st <= 0 or st >= int(memory.shape[1]):
        return memory
    sh, ro = memory[:, :st, :], memory[:, st:, :]
    if norm_type == "rms":
        sh, ro = rms_norm(sh, eps), rms_norm(ro, eps)
    elif norm_type == "layernorm":
        sh = F.layer_norm(sh, (sh.shape[-1],), eps=eps)
        ro = F.layer_norm(ro, (ro.shape[-1],), eps=eps)
    else:
        raise ValueError(f"Unsupported norm_type: {norm_type}")
    return torch.cat([sh, ro], dim=1)


def gather_chapters(bank: torch.Tensor, idx: torch.Tensor, T: int):
    """ChapteredMemoryBank.get_chapters_batched (memory_bank.py:263-293).

    Returns (memory (B, k*T, d), flat token indices (B, k*T))."""
    B, k = idx.shape
    all_idx = (idx.unsqueeze(-1) * T + torch.arange(T).view(1, 1, -1)).view(B, -1)
    mem = torch.gather(bank.unsqueeze(0).expand(B, -1, -1), 1,
                       all_idx.unsqueeze(-1).expand(-1, -1, bank.shape[-1]))
    return mem, all_idx


def weight_memory(memory: torch.Tensor, w: torch.Tensor, T: int) -> torch.Tensor:
    """model.py:689-692: every gathered row times its chapter weight."""
    ww = w.unsqueeze(-1).repeat(1, 1, T).reshape(memory.shape[0], -1, 1)
    return memory * ww


# --------------------------------------------------------------------------
# memory cross-attention (memory_transformer/memory_attention.py)
# --------------------------------------------------------------------------

def compute_qkv(h, memory, Wq, Wk, Wv, H, HK):
    """_compute_qkv (memory_attention.py:209-261), full-rank projections."""
    B, L, _ = h.shape
    if memory.dim() == 2:
        memory = memory.unsqueeze(0).expand(B, -1, -1)
    N = memory.shape[1]
    Dh = Wq.shape[0] // H
    q = linear(h, Wq).view(B, L, H, Dh)
    k = linear(memory, Wk).view(B, N, HK, Dh)
    v = linear(memory, Wv).view(B, N, HK, Dh)
    return q, k, v


def attention(q, k, v, scale=None):
    """_attention non-flash path (memory_attention.py:263-318), GQA expand."""
    H, HK = q.shape[2], k.shape[2]
    if HK != H:
        k = k.repeat_interleave(H // HK, dim=2)
        v = v.repeat_interleave(H // HK, dim=2)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    p = F.softmax(torch.matmul(qt, kt.transpose(-2, -1)) * scale, dim=-1)
    return torch.matmul(p, vt).transpose(1, 2)


def attention_weights(h, memory, Wq, Wk, H, HK, scale=None):
    """The weights forward(return_attn_weights=True) returns (memory_attention.py:437-447):
    softmax(q k^T * scale) of the recomputed q, k (GQA expanded), (B, H, L, N)."""
    q, k, _ = compute_qkv(h, memory, Wq, Wk, Wk, H, HK)
    if HK != H:
        k = k.repeat_interleave(H // HK, dim=2)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    return F.softmax(torch.matmul(q.transpose(1, 2), k.transpose(1, 2).transpose(-2, -1)) * scale, dim=-1)


def cross_attention(h, memory, Wq, Wk, Wv, Wo, H, HK, return_preproj=False):
    """MemoryCrossAttention.forward with a memory tensor (memory_attention.py:402-478)."""
    B, L, D = h.shape
    q, k, v = compute_qkv(h, memory, Wq, Wk, Wv, H, HK)
    a = attention(q, k, v).reshape(B, L, Wq.shape[0])
    if return_preproj:
        return a
    return linear(a, Wo)


def sequence_memory_layer(h, bank, Wr, br, Wq, Wk, Wv, Wo, *, H, HK, C, T, S, top_k,
                          routed_scale, normalize=False, norm_type="rms", eps=1e-6,
                          strategy="sequence", window=None, select_by="logits",
                          return_details=False):
    """Sequence-routed memory sublayer: model.py:609-692 then the memory
    cross-attention call of memory_block.py:549-558 (without the layernorm
    and residual, which belong to the caller)."""
    pooled = sequence_pool(h, strategy, window)
    logits = linear(pooled, Wr, br)
    idx, w, probs = route_sequence(logits, top_k, S, select_by=select_by)
    losses = router_losses(logits, probs, idx, C)
    ci, cw = prepend_shared_chapters(idx, w, num_chapters=C, num_shared_chapters=S,
                                     routed_scaling_factor=routed_scale)
    mem, _ = gather_chapters(bank, ci, T)
    if normalize:
        mem = normalize_shared_routed(mem, num_shared_chapters=S, tokens_per_chapter=T,
                                      norm_type=norm_type, eps=eps)
    mem = weight_memory(mem, cw, T)
    out = cross_attention(h, mem, Wq, Wk, Wv, Wo, H, HK)
    if return_details:
        return out, dict(pooled=pooled, logits=logits, probs=probs, idx=idx, w=w,
                         idx_star=ci, omega=cw, losses=losses, memory=mem)
    return out


# ---- token-level path (memory_attention.py:480-716) ----

def _gather_rows(x, tok):
    return x[tok]


def sparse_attention_unweighted(q, k, v, idx, BS, scale):
    """Joint softmax over each query's selected chapters.

    Vectorised restatement of naive_reference_unweighted
    (kernels-final/benchmark_kernels_final.py:206-236) and of the emulated
    path (memory_attention.py:856-898).  q (B,Tq,HQ,D), k/v (B,Tk,HK,D),
    idx (B,Tq,HK,S) chapter ids.  Returns (B,Tq,HQ,D) float."""
    B, Tq, HQ, D = q.shape
    HK = k.shape[2]
    G = HQ // HK
    S = idx.shape[-1]
    tok = (idx.long().unsqueeze(-1) * BS + torch.arange(BS)).reshape(B, Tq, HK, S * BS)
    out = torch.empty(B, Tq, HQ, D, dtype=q.dtype)
    for b in range(B):
        for kh in range(HK):
            kk = k[b, :, kh][tok[b, :, kh]]          # (Tq, S*BS, D)
            vv = v[b, :, kh][tok[b, :, kh]]
            for g in range(G):
                hq = kh * G + g
                sc = (q[b, :, hq].unsqueeze(1) * kk).sum(-1) * scale
                p = F.softmax(sc, dim=-1)
                out[b, :, hq] = (p.unsqueeze(-1) * vv).sum(1)
    return out


def sparse_attention_weighted(q, k, v, idx, w, BS, scale):
    """Exact per-chapter MoE: sum_s w_s softmax(q K_s^T*scale) V_s.

    Vectorised restatement of naive_reference_weighted
    (benchmark_kernels_final.py:239-294), the semantics of
    kernels-final/kernel_v4.py:1-15 and memory_attention.py:596-688.
    w (B,Tq,S)."""
    B, Tq, HQ, D = q.shape
    HK = k.shape[2]
    G = HQ // HK
    S = idx.shape[-1]
    tok = (idx.long().unsqueeze(-1) * BS + torch.arange(BS))      # (B,Tq,HK,S,BS)
    out = torch.zeros(B, Tq, HQ, D, dtype=q.dtype)
    for b in range(B):
        for kh in range(HK):
            kk = k[b, :, kh][tok[b, :, kh]]          # (Tq,S,BS,D)
            vv = v[b, :, kh][tok[b, :, kh]]
            for g in range(G):
                hq = kh * G + g
                sc = torch.einsum("td,tsjd->tsj", q[b, :, hq], kk) * scale
                p = F.softmax(sc, dim=-1)
                o = torch.einsum("tsj,tsjd->tsd", p, vv)
                out[b, :, hq] = (o * w[b].unsqueeze(-1)).sum(1)
    return out


def sparse_attention_joint_bias(q, k, v, idx, w, BS, scale, eps=1e-20):
    """Single softmax with +log(max(w, eps)) logit bias per chapter
    (benchmark_kernels_final.py:297-337, kernels-final/kernel_v5.py:1-9, :218-220)."""
    B, Tq, HQ, D = q.shape
    HK = k.shape[2]
    G = HQ // HK
    S = idx.shape[-1]
    tok = (idx.long().unsqueeze(-1) * BS + torch.arange(BS)).reshape(B, Tq, HK, S * BS)
    bias = torch.log(w.clamp_min(eps)).repeat_interleave(BS, dim=-1)   # (B,Tq,S*BS)
    out = torch.empty(B, Tq, HQ, D, dtype=q.dtype)
    for b in range(B):
        for kh in range(HK):
            kk = k[b, :, kh][tok[b, :, kh]]
            vv = v[b, :, kh][tok[b, :, kh]]
            for g in range(G):
                hq = kh * G + g
                sc = (q[b, :, hq].unsqueeze(1) * kk).sum(-1) * scale + bias[b]
                p = F.softmax(sc, dim=-1)
                out[b, :, hq] = (p.unsqueeze(-1) * vv).sum(1)
    return out


def sparse_attention_block_weighted(q, k, v, idx, bw, BS, scale):
    """v1-v3 block-weighted joint softmax: p_j = max(w_c,0) e^{s_j} / sum
    (kernels-final/kernel_v2.py:765-773 forward; :2514-2517 backward).
    bw (B,Tq,HK,S) weights per (query, kv head, slot)."""
    B, Tq, HQ, D = q.shape
    HK = k.shape[2]
    G = HQ // HK
    S = idx.shape[-1]
    tok = (idx.long().unsqueeze(-1) * BS + torch.arange(BS)).reshape(B, Tq, HK, S * BS)
    out = torch.empty(B, Tq, HQ, D, dtype=q.dtype)
    for b in range(B):
        for kh in range(HK):
            kk = k[b, :, kh][tok[b, :, kh]]
            vv = v[b, :, kh][tok[b, :, kh]]
            ww = bw[b, :, kh].clamp_min(0.0).repeat_interleave(BS, dim=-1)  # (Tq,S*BS)
            for g in range(G):
                hq = kh * G + g
                sc = (q[b, :, hq].unsqueeze(1) * kk).sum(-1) * scale
                m = sc.max(dim=-1, keepdim=True).values
                e = torch.exp(sc - m) * ww
                den = e.sum(-1, keepdim=True)
                p = torch.where(den > 0, e / torch.where(den > 0, den, torch.ones_like(den)),
                                torch.zeros_like(e))
                out[b, :, hq] = (p.unsqueeze(-1) * vv).sum(1)
    return out


# Literal loop restatements of the reference's naive kernels (small sizes only).

def naive_reference_unweighted(q, k, v, block_indices, BS, scale):
    """Loop restatement of benchmark_kernels_final.py:206-236 (B=1)."""
    _, TQ, HQ, D = q.shape
    HK = k.shape[2]
    G = HQ // HK
    out = torch.zeros((1, TQ, HQ, D), dtype=torch.float64)
    for hk in range(HK):
        for t in range(TQ):
            ch = block_indices[0, t, hk, :].long()
            tok = (ch[:, None] * BS + torch.arange(BS)[None, :]).reshape(-1)
            kk, vv = k[0, tok, hk, :].double(), v[0, tok, hk, :].double()
            for g in range(G):
                hq = hk * G + g
                sc = (q[0, t, hq, :].double() * scale) @ kk.T
                out[0, t, hq, :] = torch.softmax(sc, dim=-1) @ vv
    return out


def naive_reference_weighted(q, k, v, block_indices, chapter_weights, BS, scale):
    """Loop restatement of benchmark_kernels_final.py:239-294 (B=1)."""
    _, TQ, HQ, D = q.shape
    HK = k.shape[2]
    G = HQ // HK
    S = block_indices.shape[-1]
    out = torch.zeros((1, TQ, HQ, D), dtype=torch.float64)
    for hk in range(HK):
        for t in range(TQ):
            for g in range(G):
                hq = hk * G + g
                qt = q[0, t, hq, :].double() * scale
                acc = torch.zeros(D, dtype=torch.float64)
                for i in range(S):
                    c0 = int(block_indices[0, t, hk, i]) * BS
                    kk = k[0, c0:c0 + BS, hk, :].double()
                    vv = v[0, c0:c0 + BS, hk, :].double()
                    acc = acc + (torch.softmax(qt @ kk.T, dim=-1) @ vv) * float(chapter_weights[0, t, i])
                out[0, t, hq, :] = acc
    return out


def naive_reference_weighted_joint_bias(q, k, v, block_indices, chapter_weights, BS, scale):
    """Loop restatement of benchmark_kernels_final.py:297-337 (B=1)."""
    _, TQ, HQ, D = q.shape
    HK = k.shape[2]
    G = HQ // HK
    S = block_indices.shape[-1]
    out = torch.zeros((1, TQ, HQ, D), dtype=torch.float64)
    for hk in range(HK):
        for t in range(TQ):
            for g in range(G):
                hq = hk * G + g
                qt = q[0, t, hq, :].double() * scale
                logits, values = [], []
                for i in range(S):
                    c0 = int(block_indices[0, t, hk, i]) * BS
                    kk = k[0, c0:c0 + BS, hk, :].double()
                    logits.append(qt @ kk.T + math.log(max(float(chapter_weights[0, t, i]), 1e-20)))
                    values.append(v[0, c0:c0 + BS, hk, :].double())
                p = torch.softmax(torch.cat(logits), dim=-1)
                out[0, t, hq, :] = p @ torch.cat(values)
    return out


def naive_reference_block_weighted(q, k, v, block_indices, block_weights, BS, scale):
    """Loop form of the v1-v3 block-weighted joint softmax (B=1)."""
    _, TQ, HQ, D = q.shape
    HK = k.shape[2]
    G = HQ // HK
    S = block_indices.shape[-1]
    out = torch.zeros((1, TQ, HQ, D), dtype=torch.float64)
    for hk in range(HK):
        for t in range(TQ):
            for g in range(G):
                hq = hk * G + g
                qt = q[0, t, hq, :].double() * scale
                num = torch.zeros(D, dtype=torch.float64)
                den = 0.0
                scs = []
                for i in range(S):
                    c0 = int(block_indices[0, t, hk, i]) * BS
                    scs.append(qt @ k[0, c0:c0 + BS, hk, :].double().T)
                m = max(float(s.max()) for s in scs)
                for i in range(S):
                    c0 = int(block_indices[0, t, hk, i]) * BS
                    e = torch.exp(scs[i] - m) * max(float(block_weights[0, t, hk, i]), 0.0)
                    num = num + e @ v[0, c0:c0 + BS, hk, :].double()
                    den += float(e.sum())
                out[0, t, hq, :] = num / den if den > 0 else num * 0
    return out


def token_routed_preproj(h, shared_memory, routed_memory, idx_local, chapter_weights, T,
                         routed_scale, Wq, Wk, Wv, H, HK):
    """_forward_token_routed_attention before o_proj (memory_attention.py:480-716).

    shared: dense attention over shared rows (:549-551).  routed: per-chapter
    softmax mixed by chapter_weights (weighted, :596-688) or one joint softmax
    (chapter_weights None, :698-707); then combined + routed * routed_scale."""
    B, L, D = h.shape
    out = h.new_zeros((B, L, Wq.shape[0]))
    if shared_memory is not None and shared_memory.numel() > 0:
        out = out + cross_attention(h, shared_memory, Wq, Wk, Wv, None, H, HK, return_preproj=True)
    if routed_memory is not None and routed_memory.numel() > 0 and idx_local.shape[-1] > 0 and T > 0:
        q, k, v = compute_qkv(h, routed_memory, Wq, Wk, Wv, H, HK)
        scale = q.shape[-1] ** -0.5
        idx4 = idx_local.long().unsqueeze(2).expand(B, L, HK, idx_local.shape[-1])
        if chapter_weights is not None:
            r = sparse_attention_weighted(q, k, v, idx4, chapter_weights.to(q.dtype), T, scale)
        else:
            r = sparse_attention_unweighted(q, k, v, idx4, T, scale)
        out = out + r.reshape(B, L, -1) * routed_scale
    return out


def token_memory_layer(h, bank, Wr, br, Wq, Wk, Wv, Wo, *, H, HK, C, T, S, top_k,
                       routed_scale, normalize=False, norm_type="rms", eps=1e-6,
                       weighted=True, select_by="logits", return_details=False):
    """Token-level memory sublayer: model.py:543-607 then memory_attention.py:352-400."""
    logits = linear(h, Wr, br)
    idx, w, probs = route_token_level(logits, top_k, S, select_by=select_by)
    st = S * T
    shared = bank[:st] if st > 0 else None
    routed = bank[st:] if st < bank.shape[0] else None
    if normalize and shared is not None and routed is not None and shared.numel() > 0 and routed.numel() > 0:
        merged = normalize_shared_routed(torch.cat([shared, routed], 0).unsqueeze(0),
                                         num_shared_chapters=S, tokens_per_chapter=T,
                                         norm_type=norm_type, eps=eps).squeeze(0)
        shared, routed = merged[:st], merged[st:]
    pre = token_routed_preproj(h, shared, routed, idx - S, w if weighted else None, T,
                               routed_scale, Wq, Wk, Wv, H, HK)
    out = linear(pre, Wo)
    if return_details:
        losses = router_losses(logits.reshape(-1, C), probs.reshape(-1, C),
                               idx.reshape(-1, idx.shape[-1]), C)
        return out, dict(logits=logits, probs=probs, idx=idx, w=w, losses=losses)
    return out


def decode_step(h_t, bank, idx_star, omega, Wq, Wk, Wv, Wo, *, H, HK, T,
                normalize=False, norm_type="rms", eps=1e-6, S=1):
    """One decode step (L=1) of the sequence-routed layer with fixed (I*, omega):
    the L=1 case of sequence_memory_layer (model.py:677-692 + memory_attention)."""
    mem, _ = gather_chapters(bank, idx_star, T)
    if normalize:
        mem = normalize_shared_routed(mem, num_shared_chapters=S, tokens_per_chapter=T,
                                      norm_type=norm_type, eps=eps)
    mem = weight_memory(mem, omega, T)
    return cross_attention(h_t, mem, Wq, Wk, Wv, Wo, H, HK)


def masked_mean(states: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """model.py:468-493: mean over dim 1 ignoring mask == 0 positions; a longer mask is aligned
    on its rightmost states.shape[1] columns; the count is clamped to >= 1."""
    if mask is None:
        return states.mean(dim=1)
    if mask.shape[1] != states.shape[1]:
        mask = mask[:, -states.shape[1]:]
    m = mask.to(states.dtype).unsqueeze(-1)
    return (states * m).sum(dim=1) / m.sum(dim=1).clamp(min=1.0)


def inference_route(strategy: str, hidden: torch.Tensor, cache: Optional[torch.Tensor], Wr, br, *, top_k: int,
                    num_shared: int, num_chapters: int, routed_scale: float, window: int,
                    mask: Optional[torch.Tensor] = None, prefill: bool = False,
                    select_by_logits: Optional[torch.Tensor] = None):
    """One routing decision of MemoryTransformer.forward at inference with a decode cache
    (model.py:609-661, then the prepend of :663-670).  ``hidden`` is the call's hidden states
    (the prompt at prefill, (B, 1, d) at a step), ``cache`` the rolling window kept between
    calls.  Returns (pooled, logits, chapter ids, omega, new cache).

      sequence / sequence-rolling: the router on ``hidden`` (router.py:96-107, :158-195);
      hybrid at prefill: the masked mean of the prompt, whose last ``window`` states start the
        window (:635-642);
      rolling, and hybrid after prefill: cat(window, hidden)[-window:], masked mean (:643-654);
      then softmax -> shared-prefix mask -> renorm -> top-k -> renorm (router.py:114-149 and
      _select_routed_chapters_from_probs, model.py:331-354, the same chain).
    ``select_by_logits``: logits to select on (the tie rule of ``route_sequence``); default the
    logits computed here."""
    if strategy in ("sequence", "sequence-rolling", "sequence_rolling"):
        pooled = sequence_pool(hidden, "sequence" if strategy == "sequence" else strategy, window)
        new_cache = cache
    elif strategy == "hybrid" and prefill:
        pooled = masked_mean(hidden, mask)
        new_cache = hidden[:, -window:]
    elif strategy in ("rolling", "hybrid"):
        combined = hidden if (cache is None or prefill) else torch.cat([cache, hidden], dim=1)
        if combined.shape[1] > window:
            combined = combined[:, -window:]
        pooled = masked_mean(combined, mask)
        new_cache = combined
    else:
        raise ValueError(f"Unknown routing_strategy_inference: {strategy}")
    logits = linear(pooled, Wr, br)
    z = logits if select_by_logits is None else select_by_logits
    idx, _, _ = route_sequence(z, top_k, num_shared)
    probs = F.softmax(logits, dim=-1)
    p = probs.clone()
    S = max(0, min(int(num_shared), num_chapters))
    if S > 0:
        p[:, :S] = 0.0
    p = p / p.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    w = torch.gather(p, -1, idx)
    w = w / w.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    ci, cw = prepend_shared_chapters(idx, w, num_chapters=num_chapters, num_shared_chapters=num_shared,
                                     routed_scaling_factor=routed_scale)
    return pooled, logits, ci, cw, new_cache


def moe_with_routing(h, memory, chapter_indices, chapter_weights, T, Wq, Wk, Wv, Wo, H, HK):
    """MemoryCrossAttentionWithRouting.forward (memory_attention.py:963-1054)."""
    B = h.shape[0]
    if memory.dim() == 2:
        sel, _ = gather_chapters(memory, chapter_indices, T)
    else:
        sel = memory
    if chapter_weights is not None:
        acc = h.new_zeros(h.shape)
        for i in range(chapter_indices.shape[1]):
            out = cross_attention(h, sel[:, i * T:(i + 1) * T], Wq, Wk, Wv, Wo, H, HK)
            acc = acc + out * chapter_weights[:, i].view(B, 1, 1)
        return acc
    return cross_attention(h, sel, Wq, Wk, Wv, Wo, H, HK)


# --------------------------------------------------------------------------
# bank optimizer (training/trainer.py:309-392 builds it, :876-889 steps it)
# --------------------------------------------------------------------------
# The reference steps every parameter, the bank (memory_bank.py:62) included, with
# torch.optim.AdamW (a third-party routine: torch >= 2.0, requirements.txt:14; uv.lock pins
# nothing) after accelerator.clip_grad_norm_, i.e. torch.nn.utils.clip_grad_norm_ with the
# default norm_type 2.  Restated from the published AdamW algorithm (decoupled weight decay,
# bias-corrected moments, amsgrad off) in the operation order of torch's implementation.

def adamw_step(p: torch.Tensor, g: torch.Tensor, m: torch.Tensor, v: torch.Tensor, step: int,
               lr: float, betas=(0.9, 0.999), eps: float = 1e-8, weight_decay: float = 1e-2) -> None:
    """One AdamW step in place on (p, m, v); ``step`` is the 1-based step number after this
    step's increment (torch's ``state['step']``)."""
    b1, b2 = betas
    p.mul_(1 - lr * weight_decay)
    m.lerp_(g, 1 - b1)
    v.mul_(b2).addcmul_(g, g, value=1 - b2)
    bc1 = 1 - b1 ** step
    bc2 = 1 - b2 ** step
    denom = (v.sqrt() / math.sqrt(bc2)).add_(eps)
    p.addcdiv_(m, denom, value=-lr / bc1)


def clip_grad_norm(grads, max_norm: float) -> torch.Tensor:
    """torch.nn.utils.clip_grad_norm_ (norm_type 2) on a list of gradients, in place: the
    total norm is the 2-norm of the per-tensor 2-norms; every gradient is multiplied by
    min(1, max_norm / (total + 1e-6)).  Returns the total norm."""
    total = torch.linalg.vector_norm(torch.stack([torch.linalg.vector_norm(g, 2) for g in grads]), 2)
    coef = torch.clamp(max_norm / (total + 1e-6), max=1.0)
    for g in grads:
        g.mul_(coef)
    return total


# --------------------------------------------------------------------------
# caller side: the memory sublayer of MemoryTransformerBlock
# --------------------------------------------------------------------------

def block_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm.forward (memory_block.py:26-28): x / sqrt(mean(x^2) + eps) * weight."""
    rms = torch.sqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return x / rms * weight


def memory_sublayer(h, norm_weight, norm_bias, eps, use_rms_norm, memory, Wq, Wk, Wv, Wo, H, HK):
    """The memory lines of MemoryTransformerBlock.forward (memory_block.py:549-558):
    residual + memory_attn(memory_layernorm(h)); memory (B, N, d) is the already gathered,
    weighted memory (model.py:677-692).  LayerNorm is nn.LayerNorm (F.layer_norm)."""
    if use_rms_norm:
        x = block_rms_norm(h, norm_weight, eps)
    else:
        x = F.layer_norm(h, (h.shape[-1],), norm_weight, norm_bias, eps)
    return h + cross_attention(x, memory, Wq, Wk, Wv, Wo, H, HK)
