"""``ops/triton/rope.py:150-170`` (``apply_rope_triton``): RoPE on [B,H,S,D] q and k."""
import torch

from qwen3_triton.kernels import _ops


def _check(x, cos, sin):
    if not x.is_cuda or not cos.is_cuda or not sin.is_cuda:
        raise ValueError("rope requires ROCm tensors")
    if x.ndim != 4 or cos.ndim != 3 or sin.shape != cos.shape:
        raise ValueError("expected x=[batch,heads,seq,head_dim] and cos/sin=[batch,seq,head_dim]")
    b, _, s, d = x.shape
    if cos.shape != (b, s, d):
        raise ValueError("cos/sin shape must match x batch, sequence, and head_dim")
    if d % 2:
        raise ValueError("head_dim must be even")
    if cos.dtype != x.dtype or sin.dtype != x.dtype:
        raise TypeError("cos/sin must have the dtype of x")


def _one(x, cos, sin, backward):
    _check(x, cos, sin)
    return _ops.rope_apply(x.contiguous(), cos.contiguous(), sin.contiguous(), layout=1, backward=backward)


class _RoPEFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, cos, sin):
        ctx.save_for_backward(cos, sin)
        return _one(q, cos, sin, False), _one(k, cos, sin, False)

    @staticmethod
    def backward(ctx, grad_q, grad_k):
        cos, sin = ctx.saved_tensors
        gq = _one(grad_q, cos, sin, True) if grad_q is not None else None
        gk = _one(grad_k, cos, sin, True) if grad_k is not None else None
        return gq, gk, None, None


def apply_rope_triton(q, k, cos, sin):
    return _RoPEFunction.apply(q, k, cos, sin)
