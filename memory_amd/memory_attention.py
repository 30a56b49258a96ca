"""MemoryCrossAttention with the reference's module API, on libmoc kernels.

Mirrors memory_transformer/memory_attention.py:45-898 for full-rank
projections (q_proj/k_proj/v_proj/o_proj, bias-free, GQA-capable).  The
projections of the query side and the output are plain GEMMs (nn.Linear); the
memory side (gather, optional row norm, K/V projection of each distinct
chapter, routed attention and its backward) runs in the HIP kernels.

Three ways to call forward, all with the reference's return value
``(output (B, L, hidden_dim), None)``:
  * ``memory=`` a (N, d) or (B, N, d) tensor, N a multiple of 64: dense
    attention over it (memory_attention.py:402-478).  The rows are treated as
    64-row chapters of weight 1; a 2-D memory is projected once for the batch.
  * ``routed_memory_state=`` the fused sequence-level path: the bank, the
    selected chapters (shared prefix included) and their weights omega.  It
    computes exactly the reference's gather -> (normalise) -> x omega ->
    attention chain of memory_transformer/model.py:674-692 without
    materialising the gathered memory.
  * ``token_routing_state=`` the token-level path (memory_attention.py:480-716):
    dense shared chapters plus routed chapters per token, combined MoE-style
    (per-chapter softmax mixed by the router weights) or jointly.
"""

from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn as nn

from . import ops
from .token_routing_kernel import normalize_kernel_version
from ._half import float16_via_float32

try:
    from torch.utils.checkpoint import checkpoint as torch_checkpoint
except Exception:  # pragma: no cover
    torch_checkpoint = None

CHAPTER_TOKENS = 64  # chapter tile height of the kernels


class MemoryCrossAttention(nn.Module):
    def __init__(self, hidden_dim: int, num_heads: int, num_kv_heads: Optional[int] = None,
                 memory_dim: Optional[int] = None, use_low_rank_projections: bool = False,
                 projection_rank: Optional[int] = None, reduced_dim_mode: bool = False,
                 reduced_dim: Optional[int] = None, wo_init_zero: bool = True, dropout: float = 0.0,
                 use_flash_attention: bool = True, gradient_checkpointing: bool = False):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.memory_dim = memory_dim if memory_dim is not None else hidden_dim
        self.num_heads = num_heads
        self.num_kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        if self.num_heads <= 0:
            raise ValueError(f"num_heads must be > 0, got {self.num_heads}")
        if hidden_dim % num_heads != 0:
            raise ValueError(f"hidden_dim ({hidden_dim}) must be divisible by num_heads ({num_heads})")
        if self.num_kv_heads <= 0:
            raise ValueError(f"num_kv_heads must be > 0, got {self.num_kv_heads}")
        if self.num_heads % self.num_kv_heads != 0:
            raise ValueError(f"num_heads ({self.num_heads}) must be divisible by num_kv_heads ({self.num_kv_heads})")
        if use_low_rank_projections or reduced_dim_mode:
            raise NotImplementedError(
                "memory_amd implements the full-rank projections of MemoryCrossAttention; low-rank and "
                "reduced-dim modes (memory_attention.py:150-207) are outside this build's scope")
        if dropout and dropout > 0:
            raise NotImplementedError("attention dropout is not implemented by the HIP kernels")
        self.head_dim = hidden_dim // num_heads
        self.kv_hidden_dim = self.num_kv_heads * self.head_dim
        self.num_kv_groups = self.num_heads // self.num_kv_heads
        self.scale = self.head_dim ** -0.5
        self.dropout = dropout
        self.use_flash_attention = use_flash_attention  # kept for API parity; the HIP path is always used
        self.gradient_checkpointing = gradient_checkpointing
        self.reduced_dim_mode = False
        self.use_low_rank_projections = False
        self.q_proj = nn.Linear(self.hidden_dim, self.hidden_dim, bias=False)
        self.k_proj = nn.Linear(self.memory_dim, self.kv_hidden_dim, bias=False)
        self.v_proj = nn.Linear(self.memory_dim, self.kv_hidden_dim, bias=False)
        self.o_proj = nn.Linear(self.hidden_dim, self.hidden_dim, bias=False)
        if wo_init_zero:
            nn.init.zeros_(self.o_proj.weight)
        self._qnorm = None  # a caller's norm folded into q_proj for the duration of one call

    # ------------------------------------------------------------------ helpers
    def _project_output(self, attn_output: torch.Tensor) -> torch.Tensor:
        return ops.linear(attn_output, self.o_proj.weight)

    def _queries(self, hidden_states: torch.Tensor, qnorm=None) -> torch.Tensor:
        """q_proj(hidden_states), or q_proj(norm(hidden_states)) as one fused GEMM when the caller
        hands its memory_layernorm over (``qnorm`` = (weight, bias, eps, "rms" | "layer"))."""
        B, L, _ = hidden_states.shape
        qnorm = self._qnorm if qnorm is None else qnorm
        if qnorm is not None:
            weight, bias, eps, kind = qnorm
            q = ops.norm_linear(hidden_states, weight, bias, eps, kind, self.q_proj.weight)
        else:
            q = ops.linear(hidden_states, self.q_proj.weight)
        return q.view(B, L, self.num_heads, self.head_dim)

    def _checkpointing(self) -> bool:
        return bool(self.gradient_checkpointing and self.training and torch.is_grad_enabled() and torch_checkpoint)

    def _routed(self, hidden_states, bank, idx_star, omega, num_chapters, T, norm_type, eps, q=None):
        """``q``: the queries (B, L, H, Dh) when the caller already projected them (not with
        gradient checkpointing, whose recompute projects them again)."""
        B, L, _ = hidden_states.shape
        qnorm = self._qnorm  # captured: a checkpointed recompute runs after the forward returned

        def attend(qq):
            a = ops.routed_attention(qq, bank, self.k_proj.weight, self.v_proj.weight, omega, idx_star,
                                     num_chapters=num_chapters, tokens_per_chapter=T, norm_type=norm_type, eps=eps,
                                     num_kv_heads=self.num_kv_heads)
            return a.reshape(B, L, self.hidden_dim)

        if q is not None:
            return attend(q)
        if self._checkpointing():
            return torch_checkpoint(lambda h: attend(self._queries(h, qnorm)), hidden_states, use_reentrant=False)
        return attend(self._queries(hidden_states, qnorm))

    def _dense_as_chapters(self, hidden_states: torch.Tensor, memory: torch.Tensor, q=None) -> torch.Tensor:
        """Dense attention over `memory` via the routed kernels (64-row chapters, weight 1)."""
        bank, idx, omega, C = self._dense_routing(hidden_states, memory)
        return self._routed(hidden_states, bank, idx, omega, C, CHAPTER_TOKENS, None, 0.0, q=q)

    def _dense_routing(self, hidden_states: torch.Tensor, memory: torch.Tensor):
        """`memory` as a bank of 64-row chapters, every sequence selecting all of its own with
        weight 1: (bank, chapter ids (B, N / 64), omega, number of chapters)."""
        B = hidden_states.shape[0]
        if memory.dim() not in (2, 3):
            raise ValueError(f"memory must be (N, d) or (B, N, d), got {tuple(memory.shape)}")
        N = memory.shape[-2]
        if N % CHAPTER_TOKENS != 0:
            raise ValueError(f"memory length {N} must be a multiple of {CHAPTER_TOKENS} for the HIP kernels")
        per = N // CHAPTER_TOKENS
        dev = hidden_states.device
        if memory.dim() == 2:
            bank = memory
            idx = torch.arange(per, device=dev, dtype=torch.int32).expand(B, per)
            C = per
        else:
            if memory.shape[0] != B:
                raise ValueError("batched memory must have the batch size of hidden_states")
            bank = memory.reshape(B * N, memory.shape[-1])
            idx = (torch.arange(B, device=dev, dtype=torch.int32).view(B, 1) * per
                   + torch.arange(per, device=dev, dtype=torch.int32).view(1, per))
            C = B * per
        omega = torch.ones(B, per, device=dev, dtype=torch.float32)
        return bank, idx, omega, C

    @torch.no_grad()
    def attention_weights(self, hidden_states: torch.Tensor, memory: Optional[torch.Tensor] = None,
                          routed_memory_state: Optional[Dict[str, Any]] = None) -> torch.Tensor:
        """The attention probabilities (B, H, L, N) that forward(return_attn_weights=True) returns
        (memory_attention.py:437-447: softmax(q k^T * scale) over the memory keys, recomputed after
        the forward): N = the memory rows, or the selected chapters' rows (slot-major, omega-weighted
        keys) for ``routed_memory_state``.  Computed by moc_xattn_weights from the forward's row
        log-sum-exp; no autograd."""
        if routed_memory_state is not None:
            st = routed_memory_state
            norm_type = st.get("norm_type") if st.get("normalize", False) else None
            bank, idx, omega = st["bank"], st["chapter_indices"], st["chapter_weights"]
            C, T, eps = int(st["num_chapters"]), int(st["tokens_per_chapter"]), float(st.get("eps", 1e-6))
        elif memory is not None:
            bank, idx, omega, C = self._dense_routing(hidden_states, memory)
            norm_type, T, eps = None, CHAPTER_TOKENS, 0.0
        else:
            raise ValueError("memory must be provided when token_routing_state is None.")
        q = self._queries(hidden_states)
        return ops.routed_attention_weights(q, bank, self.k_proj.weight, self.v_proj.weight, omega, idx,
                                            num_chapters=C, tokens_per_chapter=T, norm_type=norm_type, eps=eps,
                                            num_kv_heads=self.num_kv_heads)

    # ------------------------------------------------------------------ forward
    @float16_via_float32
    def forward(self, hidden_states: torch.Tensor, memory: Optional[torch.Tensor] = None,
                token_routing_state: Optional[Dict[str, Any]] = None, token_routing_kernel_version: str = "v2",
                return_attn_weights: bool = False,
                routed_memory_state: Optional[Dict[str, Any]] = None) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        if return_attn_weights and token_routing_state is not None:
            raise ValueError("return_attn_weights=True is not supported for token_routing_state path.")
        out = self._project_output(self.attention_preproj(hidden_states, memory, token_routing_state,
                                                          token_routing_kernel_version, routed_memory_state))
        if return_attn_weights:
            return out, self.attention_weights(hidden_states, memory, routed_memory_state)
        return out, None

    def attention_preproj(self, hidden_states: torch.Tensor, memory: Optional[torch.Tensor] = None,
                          token_routing_state: Optional[Dict[str, Any]] = None,
                          token_routing_kernel_version: str = "v2",
                          routed_memory_state: Optional[Dict[str, Any]] = None,
                          query_norm=None) -> torch.Tensor:
        """forward's attention output before o_proj, (B, L, hidden_dim).  ``query_norm`` =
        (weight, bias, eps, "rms" | "layer"): hidden_states are the un-normalised rows and the norm
        is applied inside the q projection (only the queries read the normalised rows)."""
        if query_norm is not None:
            # the caller's norm, folded into the q projection (MemorySublayer): every path's
            # _queries picks it up for the duration of this call
            prev, self._qnorm = self._qnorm, query_norm
            try:
                return self.attention_preproj(hidden_states, memory, token_routing_state, token_routing_kernel_version,
                                              routed_memory_state)
            finally:
                self._qnorm = prev
        if token_routing_state is not None:
            return self._forward_token_routed_attention(hidden_states, token_routing_state,
                                                        token_routing_kernel_version)
        if routed_memory_state is not None:
            st = routed_memory_state
            norm_type = st.get("norm_type") if st.get("normalize", False) else None
            return self._routed(hidden_states, st["bank"], st["chapter_indices"], st["chapter_weights"],
                                int(st["num_chapters"]), int(st["tokens_per_chapter"]), norm_type,
                                float(st.get("eps", 1e-6)))
        if memory is None:
            raise ValueError("memory must be provided when token_routing_state is None.")
        return self._dense_as_chapters(hidden_states, memory)

    def _forward_token_routed_attention(self, hidden_states: torch.Tensor, token_routing_state: Dict[str, Any],
                                        token_routing_kernel_version: str = "v2") -> torch.Tensor:
        """Token-level routed memory attention (memory_attention.py:480-716), pre o_proj."""
        st = token_routing_state
        shared_memory = st.get("shared_memory")
        routed_memory = st.get("routed_memory")
        idx = st.get("token_chapter_indices", None)
        T = int(st.get("tokens_per_chapter", 0))
        routed_scale = float(st.get("routed_scale", 1.0))
        chapter_weights = st.get("chapter_weights", None)
        version = normalize_kernel_version(st.get("kernel_version", token_routing_kernel_version))
        if idx is None:
            raise ValueError("token_routing_state must include token_chapter_indices.")
        if idx.dim() != 3:
            raise ValueError(f"token_chapter_indices must be rank-3 [B, T, topk], got shape {tuple(idx.shape)}.")
        if idx.shape[0] != hidden_states.shape[0] or idx.shape[1] != hidden_states.shape[1]:
            raise ValueError(
                "token_chapter_indices shape prefix must match hidden_states [B, T, ...]. "
                f"got hidden_states={tuple(hidden_states.shape)}, token_chapter_indices={tuple(idx.shape)}")
        B, L, _ = hidden_states.shape
        combined = None
        has_shared = shared_memory is not None and shared_memory.numel() > 0
        has_routed = routed_memory is not None and routed_memory.numel() > 0 and idx.shape[-1] > 0 and T > 0
        # the shared and the routed branches attend with the same queries: projected once (the
        # reference's _forward_attention and _compute_qkv each project them; the gradients of the
        # two uses add up in one tensor instead of two products)
        q = self._queries(hidden_states) if has_routed and not (has_shared and self._checkpointing()) else None
        if has_shared:
            combined = self._dense_as_chapters(hidden_states, shared_memory, q=q)
        if has_routed:
            if q is None:
                q = self._queries(hidden_states)
            routed = ops.token_routed_attention(q, routed_memory, self.k_proj.weight, self.v_proj.weight, idx,
                                                chapter_weights, tokens_per_chapter=T, version=version,
                                                num_kv_heads=self.num_kv_heads)
            routed = routed.reshape(B, L, self.hidden_dim) * routed_scale
            combined = routed if combined is None else combined + routed
        if combined is None:
            combined = hidden_states.new_zeros((B, L, self.hidden_dim))
        return combined


class MemoryCrossAttentionWithRouting(nn.Module):
    """Cross-attention over sequence-level routed chapters (memory_attention.py:901-1054).

    ``forward(hidden_states, memory, chapter_indices, chapter_weights=None)``:
      * ``memory`` (N, d) is the bank, chapter i of sequence b = rows
        chapter_indices[b, i] * T ... + T (:1011-1054); a (B, k*T, d) memory is already routed
        (chapter i = rows i*T ... + T of its sequence);
      * with ``chapter_weights`` (B, k): sum_i w_i * o_proj(softmax over chapter i's keys),
        one softmax per chapter (:982-1001).  o_proj is linear and bias-free, so this is
        o_proj of the weighted per-chapter combine, which runs on the token-routed kernels'
        exact MoE mode (v4 semantics) with every token of a sequence selecting its sequence's
        chapters;
      * without weights: one joint softmax over all selected keys (:1003-1009), the dense
        path of MemoryCrossAttention over the selected rows.
    Returns ``(output (B, L, hidden_dim), None)``."""

    def __init__(self, hidden_dim: int, num_heads: int, num_chapters: int, tokens_per_chapter: int, top_k: int,
                 num_kv_heads: Optional[int] = None, memory_dim: Optional[int] = None,
                 use_low_rank_projections: bool = False, projection_rank: Optional[int] = None,
                 reduced_dim_mode: bool = False, reduced_dim: Optional[int] = None, wo_init_zero: bool = True,
                 dropout: float = 0.0, use_flash_attention: bool = True):
        super().__init__()
        self.num_chapters = num_chapters
        self.tokens_per_chapter = tokens_per_chapter
        self.top_k = top_k
        self.attention = MemoryCrossAttention(
            hidden_dim=hidden_dim, num_heads=num_heads, num_kv_heads=num_kv_heads, memory_dim=memory_dim,
            use_low_rank_projections=use_low_rank_projections, projection_rank=projection_rank,
            reduced_dim_mode=reduced_dim_mode, reduced_dim=reduced_dim, wo_init_zero=wo_init_zero,
            dropout=dropout, use_flash_attention=use_flash_attention)

    def _select_chapters(self, memory: torch.Tensor, chapter_indices: torch.Tensor) -> torch.Tensor:
        """(B, k*T, d) rows of the selected chapters (memory_attention.py:1011-1054)."""
        T = int(self.tokens_per_chapter)
        B, k = chapter_indices.shape
        rows = (chapter_indices.long().unsqueeze(-1) * T
                + torch.arange(T, device=chapter_indices.device).view(1, 1, T)).reshape(B, k * T)
        return memory[rows]

    @float16_via_float32
    def forward(self, hidden_states: torch.Tensor, memory: torch.Tensor, chapter_indices: torch.Tensor,
                chapter_weights: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        attn = self.attention
        T = int(self.tokens_per_chapter)
        if T <= 0 or T % CHAPTER_TOKENS:
            raise ValueError(f"tokens_per_chapter must be a positive multiple of {CHAPTER_TOKENS} for the HIP "
                             f"kernels, got {T}")
        selected = self._select_chapters(memory, chapter_indices) if memory.dim() == 2 else memory
        if chapter_weights is None:
            return attn(hidden_states, selected)
        from .sparse_attention import FSA_topk_sparse_attention_weighted_bthd
        B, L, _ = hidden_states.shape
        k = chapter_indices.shape[1]
        if selected.shape[1] < k * T:
            raise ValueError(f"routed memory has {selected.shape[1]} rows, needs {k} chapters of {T}")
        N = selected.shape[1]
        q = attn._queries(hidden_states)
        dt = q.dtype
        kk = ops.linear(selected.to(dt), attn.k_proj.weight.to(dt)).view(B, N, attn.num_kv_heads, attn.head_dim)
        vv = ops.linear(selected.to(dt), attn.v_proj.weight.to(dt)).view(B, N, attn.num_kv_heads, attn.head_dim)
        idx = torch.arange(k, device=q.device, dtype=torch.int32).view(1, 1, k).expand(B, L, k)
        w = chapter_weights.float().view(B, 1, k).expand(B, L, k)
        o = FSA_topk_sparse_attention_weighted_bthd(q, kk, vv, idx, w, T, softmax_scale=attn.scale,
                                                    disable_causal_mask=True)
        return attn._project_output(o.reshape(B, L, attn.hidden_dim)), None
