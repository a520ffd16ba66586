"""Dense causal GQA attention, forward and backward on the HIP flash kernels.

Mirrors ``qwen3_triton/kernels/attention.py:11-50``: ``cast_tensor(x, dtype)`` and
``causal_attention(q, k, v, *, scale=None, optimized=False)`` for contiguous [B,H,S,D] Q and
grouped K/V of equal length.  Forward saves O and the fp32 row LSE; backward is delta =
rowsum(O*dO), then dQ and dK/dV kernels (the GQA group is summed inside the dK/dV kernel, no
partial buffers, no atomics).
"""
import math

import torch

from . import _ops


def cast_tensor(x, dtype):
    if not x.is_cuda or not x.is_contiguous():
        raise ValueError('Contiguous ROCm tensor required')
    return _ops.cast(x, dtype)


def check_qkv(q, k, v, *, equal_length=True):
    if q.ndim != 4 or k.ndim != 4 or v.shape != k.shape or q.shape[0] != k.shape[0] or q.shape[3] != k.shape[3] or \
            (equal_length and q.shape[2] != k.shape[2]) or q.shape[2] > k.shape[2]:
        raise ValueError('Expected equal-length [B,H,S,D] Q and grouped K/V')
    if not q.is_cuda or any(t.device != q.device or t.dtype != q.dtype or not t.is_contiguous() for t in (q, k, v)):
        raise ValueError('Same-device/dtype contiguous ROCm QKV required; no fallback')
    if q.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError('Floating point QKV required')
    b, hq, s, d = q.shape
    hk = k.shape[1]
    if min(b, hq, hk, s, d) < 1 or hq % hk or d > 256:
        raise ValueError('Nonempty supported GQA with D<=256 required')


class _Attention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, scale, optimized):
        check_qkv(q, k, v)
        o, lse = _ops.attention_fwd(q, k, v, scale)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.scale = scale
        return o

    @staticmethod
    def backward(ctx, dy):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = _ops.attention_bwd(q, k, v, o, lse, dy.contiguous(), ctx.scale)
        return dq, dk, dv, None, None


def causal_attention(q, k, v, *, scale=None, optimized=False):
    """``kernels/attention.py:49``."""
    return _Attention.apply(q, k, v, scale if scale is not None else 1. / math.sqrt(q.shape[-1]), optimized)


class _AttentionBSHD(torch.autograd.Function):
    """Causal attention on [B,S,H,D] tensors, output [B,S,Hq,D]: the kernels read the batch, head and
    position strides directly, so the module path needs no transposed copies."""

    @staticmethod
    def forward(ctx, q, k, v, scale):
        o, lse = _ops.attention_fwd(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), scale)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.scale = scale
        return o.transpose(1, 2)

    @staticmethod
    def backward(ctx, dy):
        q, k, v, o, lse = ctx.saved_tensors
        dy = dy.contiguous()
        dq, dk, dv = _ops.attention_bwd(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), o,
                                        lse, dy.transpose(1, 2), ctx.scale)
        return dq.transpose(1, 2), dk.transpose(1, 2), dv.transpose(1, 2), None


def causal_attention_bshd(q, k, v, *, scale=None):
    """q [B,S,Hq,D], k/v [B,S,Hkv,D] contiguous -> [B,S,Hq,D] (causal, GQA)."""
    if q.ndim != 4 or k.ndim != 4 or v.shape != k.shape or q.shape[:2] != k.shape[:2] or q.shape[3] != k.shape[3]:
        raise ValueError('Expected [B,S,H,D] q and grouped k/v')
    if not q.is_cuda or any(t.device != q.device or t.dtype != q.dtype or not t.is_contiguous() for t in (q, k, v)):
        raise ValueError('Same-device/dtype contiguous ROCm QKV required; no fallback')
    if q.shape[2] % k.shape[2]:
        raise ValueError('q heads must be a multiple of kv heads')
    return _AttentionBSHD.apply(q, k, v, scale if scale is not None else q.shape[-1] ** -0.5)
