"""Single-token decode through sequence-routed memory layers.

For generation with the chapters and weights fixed by the prompt (the decode
use of memory_transformer/model.py:612-692 through
MemoryCrossAttention.forward with L = 1), the K/V projection of every chapter
is computed once per layer (``MemoryDecodeCache``, 0.8 GB per layer at the
paper shape) and each step only reads the tiles of the selected chapters:
q = q_proj(h_t) -> chapter-centric partial attention (each selected tile read
once per step for all sequences that chose it) -> joint merge over the
sequence's slots -> o_proj.  Inference only (no autograd).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib as L
from . import ops
from ._lib import call, ptr, stream_ptr


class MemoryDecodeCache:
    """Per-layer K and V tiles [C][HK][64 keys][64 dims] of the whole bank (optionally row-normalised)."""

    def __init__(self, bank: torch.Tensor, wk: torch.Tensor, wv: torch.Tensor, *, num_chapters: int,
                 tokens_per_chapter: int, num_kv_heads: int, norm_type: Optional[str] = None, eps: float = 1e-6,
                 dtype: torch.dtype = torch.bfloat16):
        L.require_gpu(bank, wk, wv)
        C, T = int(num_chapters), int(tokens_per_chapter)
        self.num_chapters, self.T, self.HK, self.dtype = C, T, int(num_kv_heads), dtype
        with torch.no_grad():
            plan = ops.identity_plan(C, bank.device)
            code = ops.norm_code(norm_type)
            mean = rstd = None
            if code:
                mean, rstd = ops.row_stats(bank.contiguous(), plan, T, code, eps)
            wkv = torch.cat([wk, wv], 0).to(dtype).contiguous()
            self.k_tiles, self.v_tiles = ops.kv_project(bank.contiguous(), plan, T, wkv, self.HK, 64, mean, rstd,
                                                        dtype, ("k", "v"))

    @property
    def nbytes(self) -> int:
        return self.k_tiles.numel() * self.k_tiles.element_size() * 2

    # File format of a saved cache (safetensors): tensors ``k_tiles`` and ``v_tiles``, each
    # [num_chapters][num_kv_heads][tokens_per_chapter keys][64 dims] in the cache dtype (the
    # projected, optionally row-normalised bank, K = norm(M) Wk^T and V = norm(M) Wv^T per
    # chapter), and string metadata: format, num_chapters, tokens_per_chapter, num_kv_heads,
    # dtype.  The K/V of one memory layer; omega is applied at attention time.
    FORMAT = "moc-decode-kv/1"

    def save(self, path: str) -> None:
        from safetensors.torch import save_file
        meta = {"format": self.FORMAT, "num_chapters": str(self.num_chapters), "tokens_per_chapter": str(self.T),
                "num_kv_heads": str(self.HK), "dtype": str(self.dtype).replace("torch.", "")}
        save_file({"k_tiles": self.k_tiles.contiguous().cpu(), "v_tiles": self.v_tiles.contiguous().cpu()}, path,
                  metadata=meta)

    @classmethod
    def load(cls, path: str, device: torch.device) -> "MemoryDecodeCache":
        from safetensors import safe_open
        with safe_open(path, framework="pt", device="cpu") as f:
            meta = f.metadata() or {}
            if meta.get("format") != cls.FORMAT:
                raise ValueError(f"{path}: not a {cls.FORMAT} decode cache (format {meta.get('format')!r})")
            k, v = f.get_tensor("k_tiles"), f.get_tensor("v_tiles")
        C, T, HK = int(meta["num_chapters"]), int(meta["tokens_per_chapter"]), int(meta["num_kv_heads"])
        if tuple(k.shape) != (C, HK, T, 64) or k.shape != v.shape:
            raise ValueError(f"{path}: tile shape {tuple(k.shape)} does not match the metadata")
        return cls.from_tiles(k.to(device), v.to(device), num_chapters=C, tokens_per_chapter=T, num_kv_heads=HK)

    @classmethod
    def from_tiles(cls, k_tiles: torch.Tensor, v_tiles: torch.Tensor, *, num_chapters: int, tokens_per_chapter: int,
                   num_kv_heads: int) -> "MemoryDecodeCache":
        """A cache over already projected tiles [num_chapters][num_kv_heads][T][64]."""
        L.require_gpu(k_tiles, v_tiles)
        if k_tiles.dtype not in (torch.float32, torch.bfloat16) or v_tiles.dtype != k_tiles.dtype:
            raise ValueError("decode cache tiles must be float32 or bfloat16, both of one dtype")
        if k_tiles.shape != (num_chapters, num_kv_heads, tokens_per_chapter, 64) or v_tiles.shape != k_tiles.shape:
            raise ValueError(f"tiles of shape {tuple(k_tiles.shape)}, expected "
                             f"{(num_chapters, num_kv_heads, tokens_per_chapter, 64)}")
        self = cls.__new__(cls)
        self.num_chapters, self.T, self.HK, self.dtype = int(num_chapters), int(tokens_per_chapter), \
            int(num_kv_heads), k_tiles.dtype
        self.k_tiles, self.v_tiles = k_tiles.contiguous(), v_tiles.contiguous()
        return self


class DecodeRouting:
    """(chapter ids incl. the shared prefix, omega) of a batch of sequences and their plan.

    ``sync=True`` (routing fixed for a whole generation): the distinct-chapter count is read
    once (one synchronisation here, none per step), so each step launches exactly one wave per
    selected (chapter, kv head) tile.  ``sync=False`` (routing that changes every step,
    ``DecodeRouter``): no host read; the launches are sized for min(B * NS, C) chapters and the
    kernels read the count on the device (waves past it exit at once)."""

    def __init__(self, chapter_indices: torch.Tensor, chapter_weights: torch.Tensor, num_chapters: int,
                 sync: bool = True):
        L.require_gpu(chapter_indices, chapter_weights)
        self.idx = chapter_indices.to(torch.int32).contiguous()
        self.omega = chapter_weights.float().contiguous()
        self.B, self.NS = self.idx.shape
        self.plan = ops.chapter_plan(self.idx, num_chapters)
        self._n_unique = int(self.plan.n_uniq[0].item()) if sync else None
        self.max_units = self._n_unique if sync else min(self.B * self.NS, int(num_chapters))
        # the first 16 edges of every distinct chapter, read by the decode kernel with its plan
        # entries (instead of after them, through csr_off); -1 rows past the count
        self.row_tab = torch.empty(max(self.max_units, 1) * 16, device=self.idx.device, dtype=torch.int32)
        call("moc_decode_row_table", ptr(self.plan.n_uniq), ptr(self.plan.csr_off), ptr(self.plan.csr_edge),
             self.max_units, ptr(self.row_tab), stream_ptr(self.idx.device))

    def unique_chapters(self) -> int:
        if self._n_unique is None:
            self._n_unique = int(self.plan.n_uniq[0].item())
        return self._n_unique


def _masked_mean(states: torch.Tensor, mask: Optional[torch.Tensor]) -> torch.Tensor:
    """Mean over the sequence ignoring padding (mask == 0), the mask's rightmost positions
    aligned with the states (memory_transformer/model.py:468-493); fp32 result."""
    if mask is None:
        return ops.router_pool(states)
    if mask.dim() != 2:
        raise ValueError(f"attention_mask must be 2D (got shape {tuple(mask.shape)})")
    if mask.shape[0] != states.shape[0]:
        raise ValueError(f"attention_mask batch ({mask.shape[0]}) must match states batch ({states.shape[0]})")
    if mask.shape[1] < states.shape[1]:
        raise ValueError(f"attention_mask length ({mask.shape[1]}) must be >= states length ({states.shape[1]})")
    if mask.shape[1] != states.shape[1]:
        mask = mask[:, -states.shape[1]:]
    m = mask.to(device=states.device, dtype=torch.float32).unsqueeze(-1)
    return (states.float() * m).sum(dim=1) / m.sum(dim=1).clamp(min=1.0)


class DecodeRouter:
    """Chapter routing of one memory layer during generation, re-decided at every step
    (MemoryTransformer.forward's inference strategies, memory_transformer/model.py:609-661):

      * "sequence" / "sequence-rolling": the router on the call's own hidden states (the prompt at
        prefill, the new token at each step), pooled as ChapterRouter pools them (mean, or the
        rolling-window mean of router.py:158-195);
      * "rolling": a window of the last ``window_size`` hidden states (prompt included), mean-pooled
        (padding masked) at prefill and at every step;
      * "hybrid": the prompt's full mean at prefill (its last ``window_size`` states start the
        window), then the rolling window at every step.

    Each call returns a ``DecodeRouting`` (shared chapters prepended, routed weights scaled and
    renormalised as model.py:356-391) built without a host synchronisation, for
    ``memory_decode_step``.  ``last_logits`` keeps the router logits of the last decision (fp32)."""

    STRATEGIES = ("sequence", "sequence-rolling", "sequence_rolling", "rolling", "hybrid")

    def __init__(self, router, *, num_chapters: int, num_shared_chapters: int = 1,
                 routed_scaling_factor: float = 2.5, strategy: str = "sequence", window_size: int = 128):
        if strategy not in self.STRATEGIES:
            raise ValueError(f"Unknown routing_strategy_inference: {strategy}")
        if int(window_size) <= 0:
            raise ValueError(f"routing_window_size must be > 0, got {window_size}")
        self.router = router
        self.num_chapters = int(num_chapters)
        self.num_shared = max(0, min(int(num_shared_chapters), self.num_chapters))
        self.routed_scale = float(routed_scaling_factor)
        self.strategy = strategy
        self.window = int(window_size)
        self.cache: Optional[torch.Tensor] = None   # (B, <= window, d): the rolling window
        self.last_logits: Optional[torch.Tensor] = None

    def reset(self) -> None:
        self.cache = None
        self.last_logits = None

    def _decide(self, pooled: torch.Tensor) -> DecodeRouting:
        from .model import prepend_shared_chapters32
        r = self.router.router
        logits = ops.router_linear(pooled, r.weight, r.bias)
        self.last_logits = logits
        C, S = self.num_chapters, self.num_shared
        k = min(int(self.router.top_k), C - S)
        if k > 0:
            idx, w = ops.router_topk(logits, k, S)
        else:
            idx = torch.empty((pooled.shape[0], 0), dtype=torch.int32, device=pooled.device)
            w = torch.empty((pooled.shape[0], 0), dtype=torch.float32, device=pooled.device)
        idx_star, omega = prepend_shared_chapters32(idx, w, num_chapters=C, num_shared_chapters=S,
                                                    routed_scaling_factor=self.routed_scale)
        return DecodeRouting(idx_star, omega, C, sync=False)

    def _own_states(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if self.strategy == "sequence":
            return ops.router_pool(hidden_states)
        from .router import rolling_coefficients
        coef = rolling_coefficients(hidden_states.shape[1], self.window, hidden_states.device)
        return ops.router_pool(hidden_states, coef)

    def _window(self, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor]) -> torch.Tensor:
        combined = hidden_states if self.cache is None else torch.cat([self.cache, hidden_states], dim=1)
        if combined.shape[1] > self.window:
            combined = combined[:, -self.window:]
        self.cache = combined.detach()
        return _masked_mean(combined, attention_mask)

    @torch.no_grad()
    def prefill(self, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor] = None) -> DecodeRouting:
        """Routing of the prompt (B, P, d); starts a new window."""
        L.require_gpu(hidden_states)
        self.reset()
        if self.strategy == "hybrid":
            pooled = _masked_mean(hidden_states, attention_mask)
            self.cache = hidden_states[:, -self.window:].detach()
            return self._decide(pooled)
        if self.strategy == "rolling":
            return self._decide(self._window(hidden_states, attention_mask))
        return self._decide(self._own_states(hidden_states))

    @torch.no_grad()
    def step(self, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor] = None) -> DecodeRouting:
        """Routing of one generated token's hidden states (B, 1, d)."""
        L.require_gpu(hidden_states)
        if self.strategy in ("rolling", "hybrid"):
            return self._decide(self._window(hidden_states, attention_mask))
        return self._decide(self._own_states(hidden_states))


def decode_attention(q: torch.Tensor, cache: MemoryDecodeCache, routing: DecodeRouting) -> torch.Tensor:
    """q (B, H, 64) -> attention output (B, H, 64) over the routed chapters (joint softmax, omega-weighted)."""
    L.require_gpu(q)
    B, H, D = q.shape
    if q.dtype != cache.dtype:
        q = q.to(cache.dtype)
    q = q.contiguous()
    dt = L.dtype_code(cache.dtype)
    st = stream_ptr(q.device)
    NS = routing.NS
    E = B * NS
    o_part = torch.empty(E * H, D, device=q.device, dtype=cache.dtype)
    lse_part = torch.empty(E * H, device=q.device, dtype=torch.float32)
    pl = routing.plan
    call("moc_decode_partial", dt, ptr(q), B, H, ptr(cache.k_tiles), ptr(cache.v_tiles), cache.HK, D, cache.T,
         ptr(pl.uniq), ptr(pl.n_uniq), ptr(pl.csr_off), ptr(pl.csr_edge), routing.max_units, ptr(routing.omega), NS,
         float(D) ** -0.5, ptr(o_part), ptr(lse_part), ptr(routing.row_tab), st)
    out = torch.empty(B, H, D, device=q.device, dtype=cache.dtype)
    lse = torch.empty(B * H, device=q.device, dtype=torch.float32)
    call("moc_sparse_combine", dt, ptr(o_part), ptr(lse_part), ptr(pl.edge_u), None, 1, NS, H, B, H, 0, ptr(out),
         ptr(lse), st)
    return out


def memory_decode_step(memory_attn, hidden: torch.Tensor, cache: MemoryDecodeCache,
                       routing: DecodeRouting) -> torch.Tensor:
    """One decode step of a memory sublayer: hidden (B, 1, d) -> (B, 1, d) (before the residual)."""
    B = hidden.shape[0]
    H = memory_attn.num_heads
    with torch.no_grad():
        wq, wo = memory_attn.q_proj.weight, memory_attn.o_proj.weight
        q = ops.linear(hidden.reshape(B, -1).to(wq.dtype), wq).view(B, H, memory_attn.head_dim)
        a = decode_attention(q, cache, routing)
        return ops.linear(a.reshape(B, 1, -1).to(wo.dtype), wo)


class DecodeStepGraph:
    """The per-token decode of several memory sublayers captured once as a HIP graph
    (torch.cuda.CUDAGraph) and replayed for every generated token: one graph launch replaces
    the ~4 kernel launches per layer, and their inter-launch gaps.

    ``layers`` is a list of (memory_attn, cache, routing); ``inputs`` the per-layer hidden
    states (B, 1, d) used for the capture (their shapes and dtypes are fixed).  ``run(inputs)``
    copies new hidden states into the captured input buffers, replays, and returns the
    per-layer outputs (buffers owned by the graph, overwritten by the next replay).  The
    routing and the caches must stay alive and unchanged while the graph is used."""

    def __init__(self, layers, inputs, warmup: int = 2):
        if len(layers) != len(inputs):
            raise ValueError("one input per layer")
        self.layers = list(layers)
        self.static_in = [x.detach().clone() for x in inputs]
        stream = torch.cuda.Stream(device=self.static_in[0].device)
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                self._body()
        torch.cuda.current_stream().wait_stream(stream)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.static_out = self._body()

    def _body(self):
        return [memory_decode_step(attn, x, cache, routing)
                for (attn, cache, routing), x in zip(self.layers, self.static_in)]

    def run(self, inputs):
        """Replay with ``inputs`` (copied into the captured input buffers unless they are those
        buffers: a serving loop that writes each token's hidden states into ``static_in``
        directly replays with no copies)."""
        for buf, x in zip(self.static_in, inputs):
            if x.data_ptr() != buf.data_ptr():
                buf.copy_(x)
        self.graph.replay()
        return self.static_out
