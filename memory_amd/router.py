"""ChapterRouter with the reference's module API, running on libmoc kernels.

Mirrors memory_transformer/router.py (constructor :28-68, forward :70-156,
route_token_level :262-340, compute_total_router_loss :490-527).  Sequence
logits are computed in fp32 (mean-pool + linear kernels); per-token logits are
fp32 results of a GEMM whose operands are in the activation dtype.  The softmax /
shared-prefix mask / top-k / renormalisation chain is one HIP kernel per row with
a HIP backward.  Top-k order: logit descending, equal logits by ascending chapter id.
"""

from __future__ import annotations

import functools
from typing import Dict, Optional, Tuple

import numpy as np
import torch
import torch.nn as nn

from . import ops
from ._half import float16_via_float32


@functools.lru_cache(maxsize=64)
def _rolling_coef_np(L: int, window: int) -> np.ndarray:
    """pooled = sum_l c_l h_l for the rolling-mean pooling (router.py:158-195)."""
    c = np.zeros(L, dtype=np.float64)
    for t in range(L):
        ln = min(t + 1, window)
        c[max(0, t - window + 1): t + 1] += 1.0 / (ln * L)
    return c.astype(np.float32)


def rolling_coefficients(L: int, window: Optional[int], device) -> torch.Tensor:
    w = L if window is None else int(window)
    if w <= 0:
        raise ValueError(f"rolling_window_size must be > 0, got {window}")
    return torch.from_numpy(_rolling_coef_np(int(L), min(w, int(L)))).to(device)


def compute_router_losses(logits: torch.Tensor, probs: Optional[torch.Tensor], idx: torch.Tensor,
                          num_chapters: int) -> Dict[str, torch.Tensor]:
    """Auxiliary losses of ChapterRouter._compute_losses (router.py:197-260) on the fused
    router-loss kernels: one pass over the (rows, C) logits, the selection frequencies from
    the selected ids directly (the reference builds a (rows, k, C) one-hot for the same
    numbers, 2.15 GB at the token-level shape).  ``probs`` (the softmax of ``logits``) is
    accepted for the reference's signature and recomputed inside the kernel."""
    return ops.router_losses(logits, idx, num_chapters)


class ChapterRouter(nn.Module):
    """Top-k chapter router (memory_transformer/router.py:15-340)."""

    def __init__(self, hidden_dim: int, num_chapters: int, top_k: int = 1, routing_strategy: str = "sequence"):
        super().__init__()
        if num_chapters <= 0:
            raise ValueError(f"num_chapters must be > 0, got {num_chapters}")
        if top_k <= 0:
            raise ValueError(f"top_k must be > 0, got {top_k}")
        if top_k > num_chapters:
            raise ValueError(f"top_k ({top_k}) must be <= num_chapters ({num_chapters})")
        self.hidden_dim = hidden_dim
        self.num_chapters = num_chapters
        self.top_k = top_k
        self.routing_strategy = routing_strategy
        self.router = nn.Linear(hidden_dim, num_chapters, bias=True)
        nn.init.normal_(self.router.weight, mean=0.0, std=0.02)
        nn.init.zeros_(self.router.bias)

    # -- logits ---------------------------------------------------------------
    def sequence_logits(self, hidden_states: torch.Tensor, rolling_window_size: Optional[int] = None) -> torch.Tensor:
        if self.routing_strategy in ("sequence", "token"):
            # "token" averages per-token logits (router.py:108-112); the mean of an affine map is the
            # affine map of the mean, so it pools first.
            pooled = ops.router_pool(hidden_states)
        elif self.routing_strategy in ("sequence-rolling", "sequence_rolling"):
            if hidden_states.dim() != 3:
                raise ValueError(f"hidden_states must be 3D (B, T, D), got shape {tuple(hidden_states.shape)}")
            if hidden_states.shape[1] <= 0:
                raise ValueError("sequence length must be > 0")
            coef = rolling_coefficients(hidden_states.shape[1], rolling_window_size, hidden_states.device)
            pooled = ops.router_pool(hidden_states, coef)
        else:
            raise ValueError(f"Unknown routing_strategy: {self.routing_strategy}")
        return ops.router_linear(pooled, self.router.weight, self.router.bias)

    # -- forward --------------------------------------------------------------
    @float16_via_float32
    def forward(self, hidden_states: torch.Tensor, return_losses: bool = True, exclude_prefix_chapters: int = 0,
                rolling_window_size: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor, Dict[str, torch.Tensor]]:
        idx, w, losses = self.route_ids32(hidden_states, return_losses, exclude_prefix_chapters, rolling_window_size)
        return idx.long(), w, losses

    def route_ids32(self, hidden_states: torch.Tensor, return_losses: bool = True, exclude_prefix_chapters: int = 0,
                    rolling_window_size: Optional[int] = None):
        """forward with the chapter ids left in int32 (the kernels' index type), for callers
        that pass them straight on to the chapter plan."""
        B = hidden_states.shape[0]
        logits = self.sequence_logits(hidden_states, rolling_window_size)
        S = int(exclude_prefix_chapters)
        if S < 0 or S > self.num_chapters:
            raise ValueError(f"exclude_prefix_chapters must be in [0, {self.num_chapters}], got {S}")
        k = min(int(self.top_k), self.num_chapters - S) if S > 0 else int(self.top_k)
        if k <= 0:
            idx = torch.empty((B, 0), dtype=torch.int32, device=hidden_states.device)
            w = torch.empty((B, 0), dtype=torch.float32, device=hidden_states.device)
        else:
            idx, w = ops.router_topk(logits, k, S)
        losses = {}
        if return_losses:
            losses = compute_router_losses(logits, None, idx, self.num_chapters)
        return idx, w, losses

    def route_token_level(self, hidden_states: torch.Tensor, return_losses: bool = True,
                          exclude_prefix_chapters: int = 0, *, ids32: bool = False):
        """Per-token routing (router.py:262-340): indices (B, T, k) are global chapter ids
        (int64 as the reference returns them; ``ids32``: the kernels' int32)."""
        if hidden_states.dim() != 3:
            raise ValueError(f"hidden_states must be 3D (B, T, D), got shape {tuple(hidden_states.shape)}")
        S = int(exclude_prefix_chapters)
        if S < 0 or S > self.num_chapters:
            raise ValueError(f"exclude_prefix_chapters must be in [0, {self.num_chapters}], got {S}")
        B, T, _ = hidden_states.shape
        C = self.num_chapters
        k = min(int(self.top_k), C - S)
        if k <= 0:
            logits = ops.router_token_logits(hidden_states, self.router.weight, self.router.bias)   # (B*T, C) fp32
            idx = torch.empty((B, T, 0), dtype=torch.int32 if ids32 else torch.long, device=hidden_states.device)
            w = torch.empty((B, T, 0), dtype=torch.float32, device=hidden_states.device)
            losses = {}
            if return_losses:
                losses = compute_router_losses(logits, None, idx.reshape(B * T, 0), C)
            return idx, w, losses
        logits, idx32, w = ops.token_router(hidden_states, self.router.weight, self.router.bias, k, S)
        idx = (idx32 if ids32 else idx32.long()).view(B, T, k)
        losses = {}
        if return_losses:
            losses = compute_router_losses(logits, None, idx32, C)
        return idx, w.view(B, T, k), losses


def compute_total_router_loss(losses: Dict[str, torch.Tensor], load_balance_coef: float = 0.01,
                              auxiliary_coef: float = 0.0, z_loss_coef: float = 0.0,
                              reference_tensor: Optional[torch.Tensor] = None) -> torch.Tensor:
    """router.py:490-527."""
    if not losses:
        if reference_tensor is not None:
            return reference_tensor.new_tensor(0.0)
        return torch.tensor(0.0)
    total = next(iter(losses.values())).new_tensor(0.0)
    if "load_balance" in losses and load_balance_coef > 0:
        total = total + load_balance_coef * losses["load_balance"]
    if "auxiliary" in losses and auxiliary_coef > 0:
        total = total + auxiliary_coef * losses["auxiliary"]
    if "z_loss" in losses and z_loss_coef > 0:
        total = total + z_loss_coef * losses["z_loss"]
    return total
