"""``ops/triton/attention_backward.py:196-236`` (``attention_backward_triton``)."""
from __future__ import annotations

import math

from qwen3_triton.kernels import _ops

from .attention import _validate


def attention_backward_triton(q, k, v, grad_out, *, scale=None, lse=None):
    """dQ, dK, dV of causal GQA attention.  The HIP backward needs O for delta = rowsum(O*dO), so
    the forward is recomputed here (it also supplies LSE when none is given)."""
    _validate(q, k, v, True)
    if grad_out.shape != q.shape:
        raise ValueError("invalid q/k/grad_out shapes")
    q, k, v, grad_out = (t.contiguous() for t in (q, k, v, grad_out))
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    out, lse_new = _ops.attention_fwd(q, k, v, scale)
    lse = lse_new if lse is None else lse.contiguous()
    return _ops.attention_bwd(q, k, v, out, lse, grad_out, scale)
