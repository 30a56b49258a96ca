"""CPU oracle for the Mixture-of-Chapters memory cross-attention hot path.

TEST INFRASTRUCTURE ONLY.  This package is the checker, never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package ``memory_amd`` never imports
it and has no CPU fallback.

Every function restates the reference algorithm from its source text (cited
``path:line`` relative to the reference repository root) in plain PyTorch-CPU
(fp32/fp64) or numpy.  Nothing from the reference is imported or executed.
"""

from .moc_oracle import *  # noqa: F401,F403
