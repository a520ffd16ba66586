"""Fused per-head RMSNorm + split-half RoPE (Q/K norm of Qwen3).

Mirrors ``qwen3_triton/kernels/norm_rope.py:53-71`` (``_NormRoPE`` / ``norm_rope``): x is
[B,S,heads,D], weight [D], cos/sin [B,S,D].  Backward fuses the inverse rotation with the
RMSNorm derivative (``q3_norm_rope_bwd``) and reduces dW deterministically.
"""
import torch

from . import _ops


def _check(x, w, cos, sin, eps):
    if x.ndim != 4 or w.shape != (x.shape[-1],) or cos.shape != sin.shape or \
            cos.shape != (x.shape[0], x.shape[1], x.shape[-1]):
        raise ValueError('Expected [B,S,heads,D], [D] and [B,S,D]')
    if not x.is_cuda or any(t.device != x.device or t.dtype != x.dtype or not t.is_contiguous()
                            for t in (x, w, cos, sin)):
        raise ValueError('Matching contiguous ROCm tensors required')
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError('Floating point required')
    if x.shape[-1] % 2 or x.numel() < 1 or eps <= 0:
        raise ValueError('Even nonempty D and positive epsilon required')
    if cos.requires_grad or sin.requires_grad:
        raise ValueError('Fixed rotary buffers only')


class _NormRoPE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, cos, sin, eps):
        _check(x, w, cos, sin, eps)
        ctx.save_for_backward(x, w, cos, sin)
        ctx.eps = eps
        return _ops.norm_rope_fwd(x, w, cos, sin, eps)

    @staticmethod
    def backward(ctx, dy):
        x, w, cos, sin = ctx.saved_tensors
        dx, dw = _ops.norm_rope_bwd(x, w, cos, sin, dy.contiguous(), ctx.eps)
        return dx, dw, None, None, None


def norm_rope(x, weight, cos, sin, eps=1e-6):
    """``kernels/norm_rope.py:71``."""
    return _NormRoPE.apply(x, weight, cos, sin, eps)
