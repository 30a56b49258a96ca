"""The token-routing kernel loader's API (memory_transformer/token_routing_kernel.py:35-142),
host side only: version normalisation and errors, which function each version resolves to,
and the per-version caches."""

import pytest

from memory_amd import sparse_attention as SA
from memory_amd import token_routing_kernel as trk


@pytest.mark.parametrize("raw,want", [(None, "v2"), ("v1", "v1"), ("2", "v2"), (" V3 ", "v3"), ("kernel_v4", "v4"),
                                      ("KERNEL_V5", "v5"), (4, "v4")])
def test_normalize_kernel_version(raw, want):
    assert trk.normalize_kernel_version(raw) == want


@pytest.mark.parametrize("bad", ["v0", "v6", "kernel", "", "v2.1", "kernel-v2"])
def test_normalize_kernel_version_rejects(bad):
    with pytest.raises(ValueError, match="Unsupported token_routing_kernel_version"):
        trk.normalize_kernel_version(bad)


@pytest.mark.parametrize("version", ["v1", "v2", "v3", "v4", "v5"])
def test_unweighted_function_for_every_version(version):
    fn = trk.get_token_routing_kernel_fn(version)
    assert fn is SA.FSA_topk_sparse_attention_bthd
    assert trk.get_token_routing_kernel_fn(version) is fn          # cached


@pytest.mark.parametrize("version,want", [("v1", None), ("v2", None), ("v3", None),
                                          ("v4", "FSA_topk_sparse_attention_weighted_bthd"),
                                          ("5", "FSA_topk_sparse_attention_weighted_joint_bias_bthd")])
def test_weighted_function_per_version(version, want):
    fn = trk.get_token_routing_weighted_kernel_fn(version)
    if want is None:
        assert fn is None
    else:
        assert fn is getattr(SA, want)


def test_loader_rejects_bad_version():
    with pytest.raises(ValueError):
        trk.get_token_routing_kernel_fn("v9")
    with pytest.raises(ValueError):
        trk.get_token_routing_weighted_kernel_fn("nine")


def test_entry_points_reject_unsupported_arguments_before_any_launch():
    """block sizes that are not a multiple of the 64-token chapter, one of cu_seqlens_q /
    cu_seqlens_k without the other and a causal memory mask raise on the host (no tensor is
    touched)."""
    with pytest.raises(ValueError, match="block_size"):
        SA.FSA_topk_sparse_attention_weighted_bthd(None, None, None, None, None, 96, disable_causal_mask=True)
    with pytest.raises(ValueError, match="block_size"):
        SA.FSA_topk_sparse_attention_bthd(None, None, None, None, 32, disable_causal_mask=True)
    with pytest.raises(ValueError, match="together"):
        SA.FSA_topk_sparse_attention_bthd(None, None, None, None, 64, cu_seqlens_q=object(),
                                          disable_causal_mask=True)
    with pytest.raises(NotImplementedError):
        SA.FSA_topk_sparse_attention_bthd(None, None, None, None, 64)
