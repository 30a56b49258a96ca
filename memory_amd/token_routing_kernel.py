"""Token-routing kernel loader with the reference's API.

Mirrors memory_transformer/token_routing_kernel.py:35-142.  Where the reference
imports Triton modules kernels-final/kernel_v{1..5}.py by file path, every
version here resolves to the HIP kernels of libmoc.so:
  * get_token_routing_kernel_fn(v)          -> FSA_topk_sparse_attention_bthd
    (joint softmax over the selected chapters, optional block weights; the
    v1-v3 signature of kernels-final/kernel_v2.py:3181-3195)
  * get_token_routing_weighted_kernel_fn(v) -> FSA_topk_sparse_attention_weighted_bthd
    for v4 (exact per-chapter MoE combine, kernels-final/kernel_v4.py:1313) and
    v5 (joint softmax with a log-weight bias, kernels-final/kernel_v5.py:819);
    None for v1-v3, which have no weighted entry point.
"""

from __future__ import annotations

import threading
from typing import Callable, Dict, Optional

_KERNEL_FN_CACHE: Dict[str, Callable] = {}
_WEIGHTED_KERNEL_FN_CACHE: Dict[str, Optional[Callable]] = {}
_CACHE_LOCK = threading.Lock()


def normalize_kernel_version(version: Optional[str]) -> str:
    """Normalize user-provided kernel version to {'v1','v2','v3','v4','v5'}."""
    if version is None:
        return "v2"
    value = str(version).strip().lower()
    for v in ("1", "2", "3", "4", "5"):
        if value in {v, f"v{v}", f"kernel_v{v}"}:
            return f"v{v}"
    raise ValueError(
        f"Unsupported token_routing_kernel_version='{version}'. Expected one of: v1, v2, v3, v4, v5.")


def get_token_routing_kernel_fn(version: Optional[str]) -> Callable:
    ver = normalize_kernel_version(version)
    with _CACHE_LOCK:
        fn = _KERNEL_FN_CACHE.get(ver)
        if fn is None:
            from .sparse_attention import FSA_topk_sparse_attention_bthd as fn
            _KERNEL_FN_CACHE[ver] = fn
    return fn


def get_token_routing_weighted_kernel_fn(version: Optional[str]) -> Optional[Callable]:
    ver = normalize_kernel_version(version)
    with _CACHE_LOCK:
        if ver not in _WEIGHTED_KERNEL_FN_CACHE:
            if ver == "v4":
                from .sparse_attention import FSA_topk_sparse_attention_weighted_bthd as fn
            elif ver == "v5":
                from .sparse_attention import FSA_topk_sparse_attention_weighted_joint_bias_bthd as fn
            else:
                fn = None
            _WEIGHTED_KERNEL_FN_CACHE[ver] = fn
        return _WEIGHTED_KERNEL_FN_CACHE[ver]
