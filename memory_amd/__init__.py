"""MI355X-native Mixture-of-Chapters memory cross-attention.

Hand-written HIP kernels for gfx950 (libmoc.so, C ABI in include/moc.h) behind
Python modules that keep the reference's API: ``router.ChapterRouter``,
``memory_attention.MemoryCrossAttention``, ``token_routing_kernel`` and the
routing helpers of ``model``.  There is no CPU path: tensors must be on a ROCm
device and libmoc.so must be built (``python -m memory_amd.build``).
"""

from . import ops  # noqa: F401

__all__ = ["ops"]
