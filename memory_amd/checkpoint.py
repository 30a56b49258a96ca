"""Loading and saving the reference's checkpoints for the memory path.

* ``load_weights(path)`` — the weights-only loading of training/trainer.py:668-709: a checkpoint
  directory holding ``model.pt`` (``torch.load(..., weights_only=True)``), ``model.safetensors``
  or ``pytorch_model.bin``, or one of those files.
* ``memory_layer_indices`` / ``memory_bank_assignments`` — which layers carry a memory sublayer
  and which bank each reads (memory_transformer/config.py:327-407).
* ``MemoryStack`` — the memory part of ``MemoryTransformer`` (model.py:120-123, :267-314;
  memory_block.py:470-499) under the reference's state-dict keys:
    ``memory_banks.{b}.base_bank.memory``            (memory_bank.py:62, :192)
    ``routers.{layer}.router.{weight,bias}``          (model.py:314, router.py:64)
    ``layers.{layer}.memory_layernorm.weight[/bias]`` (memory_block.py:476)
    ``layers.{layer}.memory_attn.{q,k,v,o}_proj.weight`` (memory_attention.py:140-143)
  ``load_reference_state_dict`` takes the reference's whole ``model.pt`` state dict (backbone keys
  are returned as unused), ``reference_state_dict`` gives these keys back for saving.
"""

from __future__ import annotations

import os
from typing import Any, Dict, List, Mapping, Optional, Tuple

import torch
import torch.nn as nn

from .memory_block import MemorySublayer
from .model import prepend_shared_chapters32, split_rows, normalize_shared_routed_memory_vectors
from .router import ChapterRouter

WEIGHT_FILES = ("model.pt", "model.safetensors", "pytorch_model.bin")


def load_weights(path: str) -> Dict[str, torch.Tensor]:
    """State dict of a checkpoint directory or file, on the CPU (trainer.py:668-709: model.pt,
    then model.safetensors, then pytorch_model.bin).  Only loaders that execute nothing from
    the file are used."""
    if os.path.isdir(path):
        for name in WEIGHT_FILES:
            f = os.path.join(path, name)
            if os.path.exists(f):
                path = f
                break
        else:
            raise FileNotFoundError(f"No supported model weights found in {path} (expected one of {WEIGHT_FILES}).")
    if path.endswith(".safetensors"):
        from safetensors.torch import load_file
        return load_file(path, device="cpu")
    return torch.load(path, map_location="cpu", weights_only=True)


def _cfg(section: Any, key: str, default=None):
    if section is None:
        return default
    if isinstance(section, Mapping):
        return section.get(key, default)
    return getattr(section, key, default)


def memory_layer_indices(num_layers: int, memory: Mapping) -> List[int]:
    """config.py:327-369 (placement "all" / "first_k" / "last_k" / "every_n" / "custom" / "none")."""
    if _cfg(memory, "vanilla_mode", False) or not _cfg(memory, "use_memory_adapter", True):
        return []
    placement = _cfg(memory, "memory_layer_placement", "all")
    if placement == "none":
        return []
    if placement == "all":
        return list(range(num_layers))
    if placement == "first_k":
        return list(range(min(int(_cfg(memory, "memory_layer_k", 5)), num_layers)))
    if placement == "last_k":
        k = min(int(_cfg(memory, "memory_layer_k", 5)), num_layers)
        return list(range(num_layers - k, num_layers))
    if placement == "every_n":
        n = int(_cfg(memory, "memory_layer_n", 3))
        if n <= 0:
            raise ValueError(f"memory_layer_n must be > 0 for 'every_n' placement, got {n}")
        return list(range(0, num_layers, n))
    if placement == "custom":
        idx = _cfg(memory, "memory_layer_indices")
        if idx is None:
            raise ValueError("memory_layer_indices must be set when using 'custom' placement")
        return sorted(i for i in idx if 0 <= i < num_layers)
    raise ValueError(f"Unknown memory_layer_placement: {placement}")


def memory_bank_assignments(num_layers: int, memory: Mapping) -> Dict[int, int]:
    """config.py:371-407 (sharing "shared" / "per_layer" / "every_k_layers")."""
    layers = memory_layer_indices(num_layers, memory)
    if not layers:
        return {}
    sharing = _cfg(memory, "memory_sharing", "shared")
    if sharing == "shared":
        return {i: 0 for i in layers}
    if sharing == "per_layer":
        return {idx: i for i, idx in enumerate(layers)}
    if sharing == "every_k_layers":
        k = int(_cfg(memory, "memory_sharing_k", 2))
        if k <= 0:
            raise ValueError(f"memory_sharing_k must be > 0 for 'every_k_layers' sharing, got {k}")
        return {idx: i // k for i, idx in enumerate(layers)}
    raise ValueError(f"Unknown memory_sharing: {sharing}")


class _Bank(nn.Module):
    def __init__(self, num_tokens: int, dim: int, init_std: float):
        super().__init__()
        self.memory = nn.Parameter(torch.empty(num_tokens, dim))
        nn.init.normal_(self.memory, mean=0.0, std=init_std)


class _ChapteredBank(nn.Module):
    """ChapteredMemoryBank(StandardMemoryBank) (memory_bank.py:176-200, :45-70): the parameter
    sits at ``base_bank.memory``."""

    def __init__(self, num_tokens: int, dim: int, num_chapters: int, init_std: float):
        super().__init__()
        if num_tokens % num_chapters != 0:
            raise ValueError(f"num_tokens ({num_tokens}) must be divisible by num_chapters ({num_chapters})")
        self.base_bank = _Bank(num_tokens, dim, init_std)
        self.num_chapters = num_chapters
        self.tokens_per_chapter = num_tokens // num_chapters

    @property
    def memory(self) -> nn.Parameter:
        return self.base_bank.memory


class MemoryStack(nn.Module):
    """Banks, routers and memory sublayers of a chaptered MemoryTransformer.

    ``forward(layer_idx, block_input, hidden_states)`` runs that layer's memory sublayer:
    routing on ``block_input`` (the hidden states entering the transformer block, as
    model.py:609-692 routes) and ``hidden_states + memory_attn(memory_layernorm(hidden_states))``
    over the routed chapters (memory_block.py:549-558).  Returns (hidden_states, router_losses)."""

    def __init__(self, *, hidden_dim: int, num_layers: int, num_heads: int, num_kv_heads: Optional[int],
                 memory: Mapping, use_rms_norm: bool = True, norm_eps: float = 1e-6):
        super().__init__()
        if not _cfg(memory, "use_chapters", False):
            raise NotImplementedError("MemoryStack covers the chaptered (routed) memory path: use_chapters must be on")
        if _cfg(memory, "use_low_rank_memory", False) or _cfg(memory, "use_low_rank_projections", False):
            raise NotImplementedError("low-rank memory and projections are outside this build")
        self.hidden_dim = int(hidden_dim)
        self.memory_dim = int(_cfg(memory, "memory_dim") or hidden_dim)
        self.num_chapters = int(_cfg(memory, "num_chapters", 100))
        self.num_memory_tokens = int(_cfg(memory, "num_memory_tokens", 1024))
        self.tokens_per_chapter = self.num_memory_tokens // self.num_chapters
        self.top_k = int(_cfg(memory, "top_k_chapters", 20))
        self.num_shared_chapters = int(_cfg(memory, "num_shared_chapters", 0))
        self.routed_scaling_factor = float(_cfg(memory, "routed_scaling_factor", 1.0))
        self.normalize = bool(_cfg(memory, "normalize_shared_routed_before_mixing", False))
        self.norm_type = _cfg(memory, "shared_routed_norm_type", "rms")
        self.norm_eps = float(_cfg(memory, "shared_routed_norm_eps", 1e-6))
        self.strategy = _cfg(memory, "routing_strategy_train", "sequence")
        self.strategy_inference = _cfg(memory, "routing_strategy_inference", "sequence")
        self.window = _cfg(memory, "routing_window_size", 128)
        self.kernel_version = _cfg(memory, "token_routing_kernel_version", "v2")
        heads = _cfg(memory, "memory_num_heads") or num_heads
        kv_heads = _cfg(memory, "memory_num_kv_heads") or num_kv_heads or heads
        self.layer_indices = memory_layer_indices(num_layers, memory)
        self.bank_of = memory_bank_assignments(num_layers, memory)
        init_std = float(_cfg(memory, "memory_init_std", 0.02))
        nbanks = (max(self.bank_of.values()) + 1) if self.bank_of else 0
        self.memory_banks = nn.ModuleDict({str(b): _ChapteredBank(self.num_memory_tokens, self.memory_dim,
                                                                  self.num_chapters, init_std)
                                           for b in range(nbanks)})
        self.routers = nn.ModuleDict({str(i): ChapterRouter(hidden_dim, self.num_chapters, self.top_k,
                                                            self.strategy)
                                      for i in self.layer_indices})
        wo0 = bool(_cfg(memory, "wo_init_zero", True))
        self.layers = nn.ModuleDict({str(i): MemorySublayer(hidden_dim, heads, kv_heads, use_rms_norm=use_rms_norm,
                                                            norm_eps=norm_eps, memory_dim=self.memory_dim,
                                                            wo_init_zero=wo0)
                                     for i in self.layer_indices})

    @classmethod
    def from_config(cls, config: Mapping) -> "MemoryStack":
        """From the reference's config (the ``config.yaml`` saved beside ``model.pt``, loaded with
        ``yaml.safe_load``, or any mapping with ``model`` and ``memory`` sections)."""
        model = config["model"] if isinstance(config, Mapping) else config.model
        memory = config["memory"] if isinstance(config, Mapping) else config.memory
        return cls(hidden_dim=int(_cfg(model, "hidden_dim")), num_layers=int(_cfg(model, "num_layers")),
                   num_heads=int(_cfg(model, "num_heads")), num_kv_heads=_cfg(model, "num_kv_heads"),
                   memory=memory, use_rms_norm=bool(_cfg(model, "use_rms_norm", True)),
                   norm_eps=float(_cfg(model, "norm_eps", 1e-6)))

    @classmethod
    def from_checkpoint(cls, checkpoint_dir: str, config: Optional[Mapping] = None, strict: bool = True):
        """``config.yaml`` and the weights of a reference checkpoint directory
        (trainer.py:1038-1101 writes both)."""
        if config is None:
            import yaml
            with open(os.path.join(checkpoint_dir, "config.yaml")) as f:
                config = yaml.safe_load(f)
        stack = cls.from_config(config)
        stack.load_reference_state_dict(load_weights(checkpoint_dir), strict=strict)
        return stack

    # ------------------------------------------------------------------ keys
    def _is_memory_key(self, key: str) -> bool:
        parts = key.split(".")
        if parts[0] in ("memory_banks", "routers"):
            return True
        return (parts[0] == "layers" and len(parts) > 2 and parts[1] in self.layers
                and parts[2] in ("memory_layernorm", "memory_attn"))

    def load_reference_state_dict(self, state_dict: Mapping[str, torch.Tensor], strict: bool = True) -> List[str]:
        """Load the memory entries of a reference ``model.pt`` state dict (values are copied
        and cast to this module's dtypes).  Returns the keys that belong to the rest of the
        model (backbone); with ``strict`` every memory parameter must be present and every
        memory key must be known."""
        own = self.state_dict()
        unused, unknown = [], []
        mem = {}
        for k, v in state_dict.items():
            if self._is_memory_key(k):
                if k in own:
                    mem[k] = v
                else:
                    unknown.append(k)
            else:
                unused.append(k)
        missing = [k for k in own if k not in mem]
        if strict and (missing or unknown):
            raise KeyError(f"reference state dict does not match the memory stack: missing {missing[:8]}, "
                           f"unexpected {unknown[:8]}")
        for k, v in mem.items():
            if tuple(v.shape) != tuple(own[k].shape):
                raise ValueError(f"{k}: shape {tuple(v.shape)} in the checkpoint, {tuple(own[k].shape)} here")
        with torch.no_grad():
            for k, v in mem.items():
                own[k].copy_(v.to(own[k].dtype))
            # a bank stepped by BankAdamW: its chapters were all brought to the last step before
            # the copy (state_dict above flushes), so the loaded values are current; the bf16
            # mirror the kernels read is refreshed from them
            for opt in self._bank_optimizers():
                opt.sync_mirror()
        return unused

    def _bank_optimizers(self):
        out = []
        for b in self.memory_banks.values():
            opt = getattr(b.memory, "_moc_bank_opt", None)
            if opt is not None:
                out.append(opt)
        return out

    def state_dict(self, *args, **kwargs):
        """nn.Module.state_dict after every BankAdamW-stepped bank is brought to its last step
        (chapters not read since then still owe their lazy zero-gradient steps)."""
        for opt in self._bank_optimizers():
            opt.flush()
        return super().state_dict(*args, **kwargs)

    def reference_state_dict(self) -> Dict[str, torch.Tensor]:
        """This stack's parameters under the reference's keys (a subset of its model.pt)."""
        return {k: v.detach() for k, v in self.state_dict().items()}

    # ------------------------------------------------------------------ forward
    def bank_for(self, layer_idx: int) -> nn.Parameter:
        return self.memory_banks[str(self.bank_of[layer_idx])].memory

    def routing_strategy(self) -> str:
        """model.py:538 and :612-625: the training strategy while training; otherwise the
        inference strategy, where "rolling" / "hybrid" (which need the decode-time routing cache)
        fall back to "sequence" as they do without use_cache."""
        if self.training:
            return self.strategy
        s = self.strategy_inference
        return "sequence" if s in ("rolling", "hybrid") else s

    def forward(self, layer_idx: int, block_input: torch.Tensor, hidden_states: torch.Tensor,
                return_losses: Optional[bool] = None):
        key = str(layer_idx)
        router, sub = self.routers[key], self.layers[key]
        bank = self.bank_for(layer_idx)
        S, T = self.num_shared_chapters, self.tokens_per_chapter
        if return_losses is None:
            return_losses = self.training             # model.py:623, return_losses=self.training
        strategy = self.routing_strategy()
        if strategy == "token":
            idx, w, losses = router.route_token_level(block_input, return_losses=return_losses,
                                                      exclude_prefix_chapters=S)
            opt = getattr(bank, "_moc_bank_opt", None)
            if opt is not None:
                opt.catch_up()
            st = min(S * T, bank.shape[0])
            src = bank
            if self.normalize and 0 < st < bank.shape[0]:
                src = normalize_shared_routed_memory_vectors(bank.unsqueeze(0), num_shared_chapters=S,
                                                             tokens_per_chapter=T, norm_type=self.norm_type,
                                                             eps=self.norm_eps).squeeze(0)
            shared, routed = split_rows(src, st)
            state = {"shared_memory": shared if st > 0 else None,
                     "routed_memory": routed if st < bank.shape[0] else None,
                     "token_chapter_indices": (idx - S).to(torch.int32), "tokens_per_chapter": T,
                     "routed_scale": self.routed_scaling_factor, "kernel_version": self.kernel_version,
                     "chapter_weights": w}
            return sub(hidden_states, token_routing_state=state,
                       token_routing_kernel_version=self.kernel_version), losses
        window = self.window if strategy in ("sequence-rolling", "sequence_rolling") else None
        router.routing_strategy = strategy            # model.py:620, as the reference sets it per call
        idx, w, losses = router.route_ids32(block_input, return_losses=return_losses, exclude_prefix_chapters=S,
                                            rolling_window_size=window)
        idx_star, omega = prepend_shared_chapters32(idx, w, num_chapters=self.num_chapters, num_shared_chapters=S,
                                                    routed_scaling_factor=self.routed_scaling_factor)
        normalize = self.normalize and 0 < S < idx_star.shape[1]
        state = {"bank": bank, "chapter_indices": idx_star, "chapter_weights": omega,
                 "num_chapters": self.num_chapters, "tokens_per_chapter": T, "normalize": normalize,
                 "norm_type": self.norm_type, "eps": self.norm_eps}
        return sub(hidden_states, routed_memory_state=state), losses
