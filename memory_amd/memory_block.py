"""The memory sublayer of MemoryTransformerBlock (memory_transformer/memory_block.py:549-558,
variant A; variant B runs the same lines at :578-587):

    residual = hidden_states
    hidden_states = self.memory_layernorm(hidden_states)
    mem_output, _ = self.memory_attn(hidden_states, memory, token_routing_state=..., ...)
    hidden_states = residual + mem_output

Here the norm (RMSNorm of memory_block.py:18-28, or nn.LayerNorm) is one HIP row kernel that
writes its output straight in the q projection's dtype, and the residual add is the
accumulator input of the o_proj GEMM.  Parameter names are the block's:
``memory_layernorm.weight`` (``.bias`` for LayerNorm) and ``memory_attn.{q,k,v,o}_proj.weight``.
"""

from __future__ import annotations

from typing import Any, Dict, Optional

import torch
import torch.nn as nn

from . import ops
from .memory_attention import MemoryCrossAttention
from ._half import float16_via_float32


class RMSNorm(nn.Module):
    """memory_block.py:18-28: y = x / sqrt(mean(x^2) + eps) * weight, on the HIP row kernel."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        return ops.row_norm(x, self.weight, None, self.eps, "rms", out_dtype)


class MemorySublayer(nn.Module):
    """``residual + memory_attn(memory_layernorm(hidden_states))`` of MemoryTransformerBlock.

    Constructor arguments follow the block's (memory_block.py:431-499): ``hidden_dim``,
    ``num_heads``, ``num_kv_heads``, ``use_rms_norm``, ``norm_eps``, ``memory_dim``,
    ``wo_init_zero``, ``gradient_checkpointing``.  ``forward`` takes the memory arguments of
    MemoryCrossAttention.forward (dense ``memory``, ``token_routing_state`` or the fused
    ``routed_memory_state``) and returns the new hidden states."""

    def __init__(self, hidden_dim: int, num_heads: int, num_kv_heads: Optional[int] = None,
                 use_rms_norm: bool = True, norm_eps: float = 1e-6, memory_dim: Optional[int] = None,
                 wo_init_zero: bool = True, gradient_checkpointing: bool = False):
        super().__init__()
        self.use_rms_norm = bool(use_rms_norm)
        self.memory_layernorm = RMSNorm(hidden_dim, norm_eps) if use_rms_norm else nn.LayerNorm(hidden_dim,
                                                                                                  eps=norm_eps)
        self.memory_attn = MemoryCrossAttention(hidden_dim, num_heads, num_kv_heads, memory_dim=memory_dim,
                                                wo_init_zero=wo_init_zero,
                                                gradient_checkpointing=gradient_checkpointing)
        # memory_layernorm folded into the q projection's GEMM where the shapes allow it
        # (ops.norm_linear_supported); False runs the norm kernel ahead of the projection
        self.fuse_norm = True

    @float16_via_float32
    def forward(self, hidden_states: torch.Tensor, memory: Optional[torch.Tensor] = None,
                token_routing_state: Optional[Dict[str, Any]] = None, token_routing_kernel_version: str = "v2",
                routed_memory_state: Optional[Dict[str, Any]] = None) -> torch.Tensor:
        attn = self.memory_attn
        cdt = attn.q_proj.weight.dtype
        if cdt not in (torch.float32, torch.bfloat16):
            raise ValueError(f"memory projections in {cdt}: the HIP kernels take float32 or bfloat16")
        ln = self.memory_layernorm
        kind = "rms" if self.use_rms_norm else "layer"
        bias = None if self.use_rms_norm else ln.bias
        if self.fuse_norm and ops.norm_linear_supported(hidden_states, attn.q_proj.weight):
            # only the q projection reads the normalised rows: the norm runs inside its GEMM
            pre = attn.attention_preproj(hidden_states, memory, token_routing_state, token_routing_kernel_version,
                                         routed_memory_state, query_norm=(ln.weight, bias, ln.eps, kind))
        else:
            x = ops.row_norm(hidden_states, ln.weight, bias, ln.eps, kind, cdt)
            pre = attn.attention_preproj(x, memory, token_routing_state, token_routing_kernel_version,
                                         routed_memory_state)
        return ops.linear_residual(pre, attn.o_proj.weight, hidden_states)
