"""float16 modules on the float32 kernels.

The kernels compute in float32 or bfloat16.  A module whose forward gets float16 tensors runs
that forward on float32 copies of them and of its float16 parameters (an exact widening,
differentiable, so the gradients reach the float16 tensors) and rounds its float32 tensor
results back to float16 -- the float16 path of the reference's torch modules, computed at
float32 precision in between.
"""

from __future__ import annotations

import functools

import torch


def _any_half(obj) -> bool:
    if isinstance(obj, torch.Tensor):
        return obj.dtype == torch.float16
    if isinstance(obj, dict):
        return any(_any_half(v) for v in obj.values())
    if isinstance(obj, (list, tuple)):
        return any(_any_half(v) for v in obj)
    return False


def _widen(obj):
    if isinstance(obj, torch.Tensor):
        return obj.float() if obj.dtype == torch.float16 else obj
    if isinstance(obj, dict):
        return {k: _widen(v) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        return type(obj)(_widen(v) for v in obj)
    return obj


def _narrow(t):
    return t.to(torch.float16) if isinstance(t, torch.Tensor) and t.dtype == torch.float32 else t


def float16_via_float32(forward):
    """Decorator of an nn.Module forward (see the module docstring).  Tensors returned directly,
    or as elements of a returned tuple, are rounded to float16; dictionaries (router losses) keep
    float32."""

    @functools.wraps(forward)
    def run(self, *args, **kwargs):
        # float16 is recognised by the inputs (a float16 module called with float32 or bfloat16
        # tensors fails on their dtypes, as the torch modules do), which keeps the check off the
        # parameters on every call
        if getattr(self, "_moc_widened", False) or not _any_half((args, kwargs)):
            return forward(self, *args, **kwargs)
        wide = {n: (p.float() if p.dtype == torch.float16 else p) for n, p in self.named_parameters()}
        self._moc_widened = True
        try:
            out = torch.func.functional_call(self, wide, _widen(args), _widen(kwargs), strict=False)
        finally:
            self._moc_widened = False
        if isinstance(out, tuple):
            return tuple(_narrow(t) for t in out)
        return _narrow(out)

    return run
