"""``qwen3_triton/inference/accumulation.py``: the reference's "reference-order" BF16 linears and short
RMSNorm rows, which replay the accumulation order of one NVIDIA GPU generation's library kernels.

Its contract is: a supported shape returns the replayed result, anything else returns ``None`` without
GPU work and the caller keeps its own route (``inference/kernels.py:131-133,177-179``).  That order has
no gfx950 counterpart, so here no shape is supported: ``strategy`` names none, ``linear`` and
``short_norm`` return ``None``, and ``inference.kernels.linear`` / ``rms_norm`` (which accept the
``reference_accumulation`` switch) run their matrix-core / RMSNorm kernels.
"""


def strategy(m, n, k):
    """``accumulation.py:13-24``: the replay strategy for an (m, n, k) linear, or None."""
    return None


def linear(x, weight, *, gemv=True):
    """``accumulation.py:67-84``: a reference-order result, or None without GPU work."""
    return None


def short_norm(x, weight, eps):
    """``accumulation.py:108-119``: a reference-order short-row RMSNorm, or None outside its domain."""
    return None
