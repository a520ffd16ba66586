"""``ops/triton/attention_backward.py:196-236`` (``attention_backward_triton``)."""
from __future__ import annotations

import math

from qwen3_triton.kernels import _ops



def _validate_backward(q, k, v, grad_out):
    """The checks of ``ops/triton/attention_backward.py:173-188``, then the head size and shared dtype
    the HIP kernels take."""
    if not all(t.is_cuda for t in (q, k, v, grad_out)):
        raise ValueError("attention backward requires ROCm tensors")
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must be rank-4 tensors")
    batch, q_heads, seq_len, head_dim = q.shape
    kv_heads = k.shape[1]
    if grad_out.shape != q.shape or k.shape != (batch, kv_heads, seq_len, head_dim):
        raise ValueError("invalid q/k/grad_out shapes")
    if v.shape != k.shape or q_heads % kv_heads != 0:
        raise ValueError("invalid GQA configuration or v shape")
    if head_dim <= 0 or head_dim % 2 != 0 or head_dim > 256:
        raise ValueError("head_dim must be a positive even number <= 256")
    if any(t.dtype != q.dtype for t in (k, v, grad_out)):
        raise TypeError("q, k, v and grad_out must share a dtype")


def attention_backward_triton(q, k, v, grad_out, *, scale=None, lse=None, out=None):
    """dQ, dK, dV of causal GQA attention ([B, H, S, D] operands).

    The backward's softmax term needs delta = rowsum(O * dO) for every query row, and a row sum
    over all keys cannot be formed tile by tile.  A caller that kept the forward output passes it
    as ``out`` (with its ``lse``): then no forward work is repeated.  Without it one forward pass
    supplies O (and LSE when ``lse`` is None).  This keyword is an addition to the reference
    signature; the autograd path (``attention_triton_autograd``) always has O saved."""
    _validate_backward(q, k, v, grad_out)
    q, k, v, grad_out = (t.contiguous() for t in (q, k, v, grad_out))
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if out is None or lse is None:
        o, lse_new = _ops.attention_fwd(q, k, v, scale)
        out = o if out is None else out
        lse = lse_new if lse is None else lse
    if out.shape != q.shape:
        raise ValueError("out must have the shape of q")
    return _ops.attention_bwd(q, k, v, out.contiguous(), lse.contiguous(), grad_out, scale)
