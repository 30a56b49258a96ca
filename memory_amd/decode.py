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
    """Fixed (chapter ids incl. the shared prefix, omega) of a batch of sequences and their plan."""

    def __init__(self, chapter_indices: torch.Tensor, chapter_weights: torch.Tensor, num_chapters: int):
        L.require_gpu(chapter_indices, chapter_weights)
        self.idx = chapter_indices.to(torch.int32).contiguous()
        self.omega = chapter_weights.float().contiguous()
        self.B, self.NS = self.idx.shape
        self.plan = ops.chapter_plan(self.idx, num_chapters)
        # the routing is fixed for the whole generation: read the distinct-chapter count once
        # (one synchronisation here, none per step) so each step launches exactly one wave per
        # selected (chapter, kv head) tile instead of min(B * NS, C) chapters' worth
        self.n_unique = int(self.plan.n_uniq[0].item())
        # the first 16 edges of every distinct chapter, read by the decode kernel with its plan
        # entries (instead of after them, through csr_off)
        self.row_tab = torch.empty(self.n_unique * 16, device=self.idx.device, dtype=torch.int32)
        call("moc_decode_row_table", ptr(self.plan.n_uniq), ptr(self.plan.csr_off), ptr(self.plan.csr_edge),
             self.n_unique, ptr(self.row_tab), stream_ptr(self.idx.device))

    def unique_chapters(self) -> int:
        return self.n_unique


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
         ptr(pl.uniq), ptr(pl.n_uniq), ptr(pl.csr_off), ptr(pl.csr_edge), routing.n_unique, ptr(routing.omega), NS,
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
