"""Shared helpers for the test-suite (seeded inputs, tolerance checks)."""

import torch


def rel_max_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """max |a - b| / max |b| (b is the reference)."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = b.abs().max().item()
    return (a - b).abs().max().item() / (den if den > 0 else 1.0)


def assert_rel(a, b, tol, what=""):
    e = rel_max_err(a, b)
    assert e <= tol, f"{what}: relative max error {e:.3e} > {tol:.1e}"


def gen(seed):
    return torch.Generator().manual_seed(seed)
