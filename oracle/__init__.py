"""CPU oracle for the Qwen3 decoder operator set (TEST INFRASTRUCTURE ONLY).

This package is a plain PyTorch-CPU restatement of the reference's math
(wuyii8941/qwen3-triton, ``ops/reference/*`` and the causal-LM glue in
``model/qwen_tiny.py`` / ``qwen3_triton/kernels/loss.py`` /
``qwen3_triton/inference/*``).  It exists to *check* the HIP path.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import it; the product package never does, and it has no fallback
role: a missing HIP library is an error, never a reason to run this code.

Every function cites the reference file:line it restates.  How each one is
pinned (closed forms, invariants, brute force, third-party library routines)
is listed in ``tests/test_oracle.py``.
"""
from .reference import *  # noqa: F401,F403
