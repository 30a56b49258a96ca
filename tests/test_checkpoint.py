"""Checkpoint compatibility on the CPU: the reference's layer placement / bank sharing rules
(memory_transformer/config.py:327-407), and loading the memory entries of a reference model.pt
state dict (keys of memory_bank.py:62/:192, model.py:314, memory_block.py:476,
memory_attention.py:140-143) into MemoryStack and back.  The state dicts are built here with
the reference's key names (the reference model itself is not run)."""

import os

import pytest
import torch
import yaml

from memory_amd.checkpoint import MemoryStack, load_weights, memory_bank_assignments, memory_layer_indices


def _mem(**kw):
    base = {"use_chapters": True, "num_memory_tokens": 9 * 64, "num_chapters": 9, "top_k_chapters": 3,
            "num_shared_chapters": 1, "routed_scaling_factor": 2.5}
    base.update(kw)
    return base


@pytest.mark.parametrize("kw,layers", [
    ({"memory_layer_placement": "all"}, [0, 1, 2, 3, 4, 5]),
    ({"memory_layer_placement": "first_k", "memory_layer_k": 2}, [0, 1]),
    ({"memory_layer_placement": "last_k", "memory_layer_k": 2}, [4, 5]),
    ({"memory_layer_placement": "last_k", "memory_layer_k": 9}, [0, 1, 2, 3, 4, 5]),
    ({"memory_layer_placement": "every_n", "memory_layer_n": 4}, [0, 4]),
    ({"memory_layer_placement": "custom", "memory_layer_indices": [5, 1, 9, -1]}, [1, 5]),
    ({"memory_layer_placement": "none"}, []),
    ({"vanilla_mode": True}, []),
    ({"use_memory_adapter": False}, []),
])
def test_memory_layer_indices(kw, layers):
    assert memory_layer_indices(6, _mem(**kw)) == layers


@pytest.mark.parametrize("kw,banks", [
    ({"memory_sharing": "shared"}, {0: 0, 2: 0, 4: 0}),
    ({"memory_sharing": "per_layer"}, {0: 0, 2: 1, 4: 2}),
    ({"memory_sharing": "every_k_layers", "memory_sharing_k": 2}, {0: 0, 2: 0, 4: 1}),
])
def test_memory_bank_assignments(kw, banks):
    assert memory_bank_assignments(6, _mem(memory_layer_placement="every_n", memory_layer_n=2, **kw)) == banks


@pytest.mark.parametrize("kw", [{"memory_layer_placement": "every_n", "memory_layer_n": 0},
                                {"memory_layer_placement": "custom"},
                                {"memory_layer_placement": "sideways"}])
def test_placement_errors(kw):
    with pytest.raises(ValueError):
        memory_layer_indices(6, _mem(**kw))


def _config(use_rms=True, sharing="per_layer"):
    return {"model": {"hidden_dim": 128, "num_layers": 6, "num_heads": 2, "num_kv_heads": 2, "use_rms_norm": use_rms,
                      "norm_eps": 1e-5},
            "memory": _mem(memory_layer_placement="every_n", memory_layer_n=2, memory_sharing=sharing)}


def _reference_state_dict(cfg, seed=0):
    """A state dict with the reference's key names for the memory entries, plus backbone entries."""
    g = torch.Generator().manual_seed(seed)
    d, m = cfg["model"]["hidden_dim"], cfg["memory"]
    layers = memory_layer_indices(cfg["model"]["num_layers"], m)
    banks = memory_bank_assignments(cfg["model"]["num_layers"], m)
    sd = {"embed_tokens.weight": torch.randn(100, d, generator=g), "norm.weight": torch.randn(d, generator=g),
          "lm_head.weight": torch.randn(100, d, generator=g)}
    for i in range(cfg["model"]["num_layers"]):
        sd[f"layers.{i}.self_attn.q_proj.weight"] = torch.randn(d, d, generator=g)
        sd[f"layers.{i}.input_layernorm.weight"] = torch.randn(d, generator=g)
        sd[f"layers.{i}.mlp.up_proj.weight"] = torch.randn(4 * d, d, generator=g)
    for b in sorted(set(banks.values())):
        sd[f"memory_banks.{b}.base_bank.memory"] = torch.randn(m["num_memory_tokens"], d, generator=g)
    for i in layers:
        sd[f"routers.{i}.router.weight"] = torch.randn(m["num_chapters"], d, generator=g)
        sd[f"routers.{i}.router.bias"] = torch.randn(m["num_chapters"], generator=g)
        for p in "qkvo":
            sd[f"layers.{i}.memory_attn.{p}_proj.weight"] = torch.randn(d, d, generator=g)
        sd[f"layers.{i}.memory_layernorm.weight"] = torch.randn(d, generator=g)
        if not cfg["model"]["use_rms_norm"]:
            sd[f"layers.{i}.memory_layernorm.bias"] = torch.randn(d, generator=g)
    return sd


@pytest.mark.parametrize("fmt", ["model.pt", "model.safetensors", "pytorch_model.bin"])
@pytest.mark.parametrize("use_rms", [True, False])
def test_load_reference_checkpoint_round_trip(tmp_path, fmt, use_rms):
    cfg = _config(use_rms)
    sd = _reference_state_dict(cfg)
    if fmt.endswith(".safetensors"):
        from safetensors.torch import save_file
        save_file(sd, os.path.join(tmp_path, fmt))
    else:
        torch.save(sd, os.path.join(tmp_path, fmt))
    with open(os.path.join(tmp_path, "config.yaml"), "w") as f:
        yaml.safe_dump(cfg, f)
    stack = MemoryStack.from_checkpoint(str(tmp_path))
    back = stack.reference_state_dict()
    mem_keys = {k for k in sd if k.startswith(("memory_banks.", "routers.")) or ".memory_" in k}
    assert set(back) == mem_keys
    for k in mem_keys:
        assert torch.equal(back[k], sd[k]), k
    unused = stack.load_reference_state_dict(load_weights(str(tmp_path)))
    assert set(unused) == set(sd) - mem_keys


def test_strict_loading_errors():
    cfg = _config()
    sd = _reference_state_dict(cfg)
    stack = MemoryStack.from_config(cfg)
    bad = dict(sd)
    del bad["routers.2.router.bias"]
    with pytest.raises(KeyError):
        stack.load_reference_state_dict(bad)
    bad = dict(sd)
    bad["layers.0.memory_attn.q_proj.lora_A"] = torch.zeros(1)
    with pytest.raises(KeyError):
        stack.load_reference_state_dict(bad)
    bad = dict(sd)
    bad["memory_banks.1.base_bank.memory"] = torch.zeros(5, 128)
    with pytest.raises(ValueError):
        stack.load_reference_state_dict(bad)
    assert stack.load_reference_state_dict({k: v for k, v in sd.items() if k != "routers.2.router.bias"},
                                           strict=False)


def test_missing_weights_file(tmp_path):
    with pytest.raises(FileNotFoundError):
        load_weights(str(tmp_path))
