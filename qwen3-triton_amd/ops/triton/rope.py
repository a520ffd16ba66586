"""``ops/triton/rope.py:150-170`` (``apply_rope_triton``): RoPE on [B,H,S,D] q and k."""
import torch

from qwen3_triton.kernels import _ops


def _check(x, cos, sin, what):
    if not x.is_cuda or not cos.is_cuda or not sin.is_cuda:
        raise ValueError("rope_triton requires ROCm tensors")
    if x.ndim != 4 or cos.ndim != 3 or sin.shape != cos.shape:
        raise ValueError(f"expected {what}=[batch,heads,seq,head_dim] and cos/sin=[batch,seq,head_dim]")
    b, _, s, d = x.shape
    if cos.shape != (b, s, d):
        raise ValueError(f"cos/sin shape must match {what} batch, sequence, and head_dim")
    if d % 2:
        raise ValueError("head_dim must be even")
    if d > 65536:
        raise ValueError("head_dim is too large for this first kernel")


def _one(x, cos, sin, backward):
    """Rotated x in x's dtype.  Tables of another dtype are taken as the reference's kernel takes them
    (every operand widened to fp32, the result stored in x's dtype): the op then runs in fp32."""
    _check(x, cos, sin, "grad" if backward else "x")
    if cos.dtype == x.dtype and sin.dtype == x.dtype:
        return _ops.rope_apply(x.contiguous(), cos.contiguous(), sin.contiguous(), layout=1, backward=backward)
    f32 = lambda t: _ops.cast(t.contiguous(), torch.float32)
    return _ops.cast(_ops.rope_apply(f32(x), f32(cos), f32(sin), layout=1, backward=backward), x.dtype)


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
