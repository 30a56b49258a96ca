"""Routing glue of MemoryTransformer for the memory layers, on libmoc kernels.

Mirrors the static helpers of memory_transformer/model.py (:331-432) and the
per-memory-layer routing block of MemoryTransformer.forward (:527-692), plus
the memory sublayer call of MemoryTransformerBlock (memory_block.py:549-558,
without the caller-owned RMSNorm and residual).

``RoutedMemoryLayer`` is the fused sequence-level memory layer: router ->
shared-chapter prepend -> [gather -> optional row norm -> x omega -> K/V
projection -> joint attention] -> o_proj, where the bracket never
materialises the (B, (S+k)*T, d) gathered memory.  ``TokenRoutedMemoryLayer``
is the token-level variant (model.py:543-607 + memory_attention.py:480-716).
"""

from __future__ import annotations

from typing import Dict, Optional, Tuple

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops, seq_layer
from .memory_attention import MemoryCrossAttention
from .router import ChapterRouter, compute_router_losses, rolling_coefficients
from ._half import float16_via_float32


def select_routed_chapters_from_probs(probs: torch.Tensor, top_k: int, num_shared_chapters: int):
    """model.py:331-354: mask the shared prefix, renormalise, top-k, renormalise.

    The masked, renormalised probabilities are formed in the probabilities' dtype as the
    reference does; the router top-k kernel selects on those values directly (its selection is
    a radix select on the raw fp32 keys; ties: lower chapter id first), and the weights are
    the selected values renormalised, so gradients flow to ``probs`` as in the reference."""
    B, C = probs.shape
    S = max(0, min(int(num_shared_chapters), C))
    k = min(int(top_k), C - S)
    if k <= 0:
        return (torch.empty((B, 0), dtype=torch.long, device=probs.device),
                torch.empty((B, 0), dtype=probs.dtype, device=probs.device))
    masked = probs.clone()
    if S > 0:
        masked[:, :S] = 0.0
    masked = masked / masked.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    with torch.no_grad():
        idx, _ = ops.router_topk(masked.detach().float(), k, S)
    idx = idx.long()
    w = masked.gather(-1, idx)
    w = w / w.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    return idx, w


def prepend_shared_chapters(chapter_indices: torch.Tensor, chapter_weights: torch.Tensor, *, num_chapters: int,
                            num_shared_chapters: int, routed_scaling_factor: float):
    """model.py:356-391 (prepend kernel + its backward)."""
    idx_star, omega = prepend_shared_chapters32(chapter_indices, chapter_weights, num_chapters=num_chapters,
                                                num_shared_chapters=num_shared_chapters,
                                                routed_scaling_factor=routed_scaling_factor)
    return idx_star.long(), omega


def prepend_shared_chapters32(chapter_indices: torch.Tensor, chapter_weights: torch.Tensor, *, num_chapters: int,
                              num_shared_chapters: int, routed_scaling_factor: float):
    """prepend_shared_chapters with int32 chapter ids (no conversion kernels on the layer's
    own path)."""
    S = max(0, min(int(num_shared_chapters), int(num_chapters)))
    if S <= 0:
        return chapter_indices.to(torch.int32), chapter_weights
    return ops.prepend_shared(chapter_indices, chapter_weights, S, routed_scaling_factor)


def normalize_shared_routed_memory_vectors(memory: torch.Tensor, *, num_shared_chapters: int,
                                           tokens_per_chapter: int, norm_type: str, eps: float) -> torch.Tensor:
    """model.py:393-432 on a materialised (B, N, d) memory (the unfused glue).

    The fused path applies the same per-row normalisation inside the gather
    prologue of the K/V projection kernel."""
    if memory.dim() != 3:
        raise ValueError(f"memory must be 3D (B, T, D), got shape {tuple(memory.shape)}")
    if tokens_per_chapter <= 0:
        return memory
    st = min(max(0, int(num_shared_chapters)) * int(tokens_per_chapter), int(memory.shape[1]))
    if st <= 0 or st >= int(memory.shape[1]):
        return memory
    if norm_type == "rms":
        return memory / memory.pow(2).mean(dim=-1, keepdim=True).add(eps).sqrt()
    if norm_type == "layernorm":
        return F.layer_norm(memory, (memory.shape[-1],), eps=eps)
    raise ValueError(f"Unsupported norm_type: {norm_type}")


class _SplitRows(torch.autograd.Function):
    """(x[:n], x[n:]) whose backward writes both row-block gradients into one new tensor
    with a single concatenation (autograd's slice backward zero-fills a full-size
    gradient per slice, copies into it and sums the two)."""

    @staticmethod
    def forward(ctx, x, n):
        ctx.n, ctx.shape = n, x.shape
        return x[:n], x[n:]

    @staticmethod
    def backward(ctx, ga, gb):
        n, shape = ctx.n, ctx.shape
        ref = ga if ga is not None else gb
        # the token path writes its gradient into the tail of a whole-shape buffer that it marks
        # (sparse_attention._rows_grad sets ``_moc_rows_tail`` on it): fill the head rows of that
        # buffer and return it.  Any other view (e.g. from cat's backward) takes the copy below.
        base = None if gb is None else gb._base
        if base is not None and getattr(base, "_moc_rows_tail", None) == n and base.shape == shape \
                and base.dtype == gb.dtype and base.is_contiguous() \
                and gb.storage_offset() - base.storage_offset() == n * math.prod(shape[1:]):
            if ga is None:
                base[:n].zero_()
            else:
                base[:n].copy_(ga)
            return base, None
        if ga is None:
            ga = ref.new_zeros((n,) + tuple(shape[1:]))
        if gb is None:
            gb = ref.new_zeros((shape[0] - n,) + tuple(shape[1:]))
        out = torch.empty(shape, device=ref.device, dtype=ref.dtype)
        out[:n].copy_(ga)       # two device copies (faster than torch.cat's kernel here)
        out[n:].copy_(gb)
        return out, None


def split_rows(x: torch.Tensor, n: int):
    if not x.requires_grad:
        return x[:n], x[n:]
    return _SplitRows.apply(x, n)


class RoutedMemoryLayer(nn.Module):
    """One sequence-routed memory sublayer (router + memory cross-attention).

    Parameter names follow the reference state dict: ``router.router.{weight,bias}``
    (model.py:314 / router.py:64) and ``memory_attn.{q,k,v,o}_proj.weight``
    (memory_block.py:476 / memory_attention.py:140-143).  The bank is passed to
    forward (the reference shares one bank between memory layers)."""

    def __init__(self, hidden_dim: int, num_heads: int, num_chapters: int, tokens_per_chapter: int, top_k: int,
                 num_shared_chapters: int = 1, routed_scaling_factor: float = 2.5, num_kv_heads: Optional[int] = None,
                 normalize_shared_routed_before_mixing: bool = False, shared_routed_norm_type: str = "rms",
                 shared_routed_norm_eps: float = 1e-6, routing_strategy: str = "sequence",
                 routing_window_size: Optional[int] = None, wo_init_zero: bool = True,
                 gradient_checkpointing: bool = False):
        super().__init__()
        self.num_chapters = int(num_chapters)
        self.tokens_per_chapter = int(tokens_per_chapter)
        self.num_shared_chapters = int(num_shared_chapters)
        self.routed_scaling_factor = float(routed_scaling_factor)
        self.normalize = bool(normalize_shared_routed_before_mixing)
        self.norm_type = shared_routed_norm_type
        self.norm_eps = float(shared_routed_norm_eps)
        self.routing_window_size = routing_window_size
        self.router = ChapterRouter(hidden_dim, num_chapters, top_k, routing_strategy)
        self.memory_attn = MemoryCrossAttention(hidden_dim, num_heads, num_kv_heads, wo_init_zero=wo_init_zero,
                                                gradient_checkpointing=gradient_checkpointing)
        # run the whole layer as one autograd function (memory_amd.seq_layer) where it applies;
        # False keeps the per-op autograd functions (router, q_proj, attention, o_proj)
        self.fused = True

    def route(self, hidden_states: torch.Tensor, return_losses: bool = True):
        idx_star, omega, losses = self._route32(hidden_states, return_losses)
        return idx_star.long(), omega, losses

    def _route32(self, hidden_states: torch.Tensor, return_losses: bool = True):
        idx, w, losses = self.router.route_ids32(hidden_states, return_losses=return_losses,
                                                 exclude_prefix_chapters=self.num_shared_chapters,
                                                 rolling_window_size=self.routing_window_size)
        idx_star, omega = prepend_shared_chapters32(idx, w, num_chapters=self.num_chapters,
                                                    num_shared_chapters=self.num_shared_chapters,
                                                    routed_scaling_factor=self.routed_scaling_factor)
        return idx_star, omega, losses

    def _fused(self, hidden_states: torch.Tensor, bank: torch.Tensor):
        """The whole layer as one autograd function (memory_amd.seq_layer) when it applies."""
        if not self.fused:
            return None
        attn = self.memory_attn
        strategy = self.router.routing_strategy
        S = self.num_shared_chapters
        C = self.num_chapters
        if strategy not in ("sequence", "token", "sequence-rolling", "sequence_rolling"):
            return None
        if attn.gradient_checkpointing and self.training:
            return None
        k = min(int(self.router.top_k), C - S)
        if not seq_layer.supported(hidden_states, bank, attn.q_proj.weight, attn.o_proj.weight,
                                   self.router.router.weight, S, k, C, self.tokens_per_chapter):
            return None
        coef = None
        if strategy in ("sequence-rolling", "sequence_rolling"):
            coef = rolling_coefficients(hidden_states.shape[1], self.routing_window_size, hidden_states.device)
        normalize = self.normalize and 0 < S < S + k
        return seq_layer.seq_routed_layer(
            hidden_states, bank, self.router.router.weight, self.router.router.bias, attn.q_proj.weight,
            attn.k_proj.weight, attn.v_proj.weight, attn.o_proj.weight, num_chapters=C,
            tokens_per_chapter=self.tokens_per_chapter, num_shared=S, top_k=k,
            routed_scale=self.routed_scaling_factor, num_heads=attn.num_heads, num_kv_heads=attn.num_kv_heads,
            norm_type=self.norm_type if normalize else None, eps=self.norm_eps, coef=coef)

    @float16_via_float32
    def forward(self, hidden_states: torch.Tensor, bank: torch.Tensor,
                return_losses: bool = True) -> Tuple[torch.Tensor, Dict[str, torch.Tensor]]:
        fused = self._fused(hidden_states, bank)
        if fused is not None:
            out, logits, idx, _, _ = fused
            losses = compute_router_losses(logits, None, idx, self.num_chapters) if return_losses else {}
            return out, losses
        idx_star, omega, losses = self._route32(hidden_states, return_losses)
        NS = idx_star.shape[1]
        # model.py:402-405: normalisation only mixes when both the shared and routed slices are non-empty
        normalize = self.normalize and 0 < self.num_shared_chapters < NS
        state = {"bank": bank, "chapter_indices": idx_star, "chapter_weights": omega,
                 "num_chapters": self.num_chapters, "tokens_per_chapter": self.tokens_per_chapter,
                 "normalize": normalize, "norm_type": self.norm_type, "eps": self.norm_eps}
        out, _ = self.memory_attn(hidden_states, routed_memory_state=state)
        return out, losses


class TokenRoutedMemoryLayer(nn.Module):
    """Token-level memory sublayer (model.py:543-607 + memory_attention.py:480-716).

    Every token routes to its own top-k routed chapters; the shared prefix is attended
    densely; routed chapters are combined MoE-style (per-chapter softmax mixed by the
    router weights, the reference's default since its glue always passes
    ``chapter_weights``) or jointly when ``weighted`` is False."""

    def __init__(self, hidden_dim: int, num_heads: int, num_chapters: int, tokens_per_chapter: int, top_k: int,
                 num_shared_chapters: int = 1, routed_scaling_factor: float = 2.5, num_kv_heads: Optional[int] = None,
                 normalize_shared_routed_before_mixing: bool = False, shared_routed_norm_type: str = "rms",
                 shared_routed_norm_eps: float = 1e-6, weighted: bool = True, kernel_version: str = "v4",
                 wo_init_zero: bool = True):
        super().__init__()
        self.num_chapters = int(num_chapters)
        self.tokens_per_chapter = int(tokens_per_chapter)
        self.num_shared_chapters = max(0, min(int(num_shared_chapters), int(num_chapters)))
        self.routed_scaling_factor = float(routed_scaling_factor)
        self.normalize = bool(normalize_shared_routed_before_mixing)
        self.norm_type = shared_routed_norm_type
        self.norm_eps = float(shared_routed_norm_eps)
        self.weighted = bool(weighted)
        self.kernel_version = kernel_version
        self.router = ChapterRouter(hidden_dim, num_chapters, top_k, "token")
        self.memory_attn = MemoryCrossAttention(hidden_dim, num_heads, num_kv_heads, wo_init_zero=wo_init_zero)

    @float16_via_float32
    def forward(self, hidden_states: torch.Tensor, bank: torch.Tensor,
                return_losses: bool = True) -> Tuple[torch.Tensor, Dict[str, torch.Tensor]]:
        S, T = self.num_shared_chapters, self.tokens_per_chapter
        idx, w, losses = self.router.route_token_level(hidden_states, return_losses=return_losses,
                                                       exclude_prefix_chapters=S, ids32=True)
        opt = getattr(bank, "_moc_bank_opt", None)
        if opt is not None:
            opt.catch_up()   # every chapter is projected: bring the whole bank to the last step
        st = min(S * T, bank.shape[0])
        src = bank
        if self.normalize and 0 < st < bank.shape[0]:
            src = normalize_shared_routed_memory_vectors(bank.unsqueeze(0), num_shared_chapters=S,
                                                         tokens_per_chapter=T, norm_type=self.norm_type,
                                                         eps=self.norm_eps).squeeze(0)
        shared, routed = split_rows(src, st)
        shared = shared if st > 0 else None
        routed = routed if st < bank.shape[0] else None
        state = {"shared_memory": shared, "routed_memory": routed,
                 "token_chapter_indices": idx - S if S else idx, "tokens_per_chapter": T,
                 "routed_scale": self.routed_scaling_factor, "kernel_version": self.kernel_version,
                 "chapter_weights": w if self.weighted else None}
        out, _ = self.memory_attn(hidden_states, token_routing_state=state)
        return out, losses
