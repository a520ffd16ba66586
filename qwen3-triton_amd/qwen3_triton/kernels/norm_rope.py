"""Fused per-head RMSNorm + split-half RoPE (Q/K norm of Qwen3).

Mirrors ``qwen3_triton/kernels/norm_rope.py:53-71`` (``_NormRoPE`` / ``norm_rope``): x is
[B,S,heads,D], weight [D], cos/sin [B,S,D].  Backward fuses the inverse rotation with the
RMSNorm derivative (``q3_norm_rope_bwd``) and reduces dW deterministically.  ``norm_rope_pair`` is
the query/key pair of one layer (``ops/triton/fused_qk_norm_rope.py:237-273``) in one launch per
direction.
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
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16) or x.shape[-1] % 2 or x.numel() < 1 or eps <= 0:
        raise ValueError('Floating point, even nonempty D and positive epsilon required')
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


class _NormRoPEPair(torch.autograd.Function):
    """q [B,S,Hq,D] and k [B,S,Hk,D] with their own weights and the shared tables: one launch per
    direction (``q3_norm_rope_qk_fwd`` / ``_bwd``), or one per tensor outside the vector path."""

    @staticmethod
    def forward(ctx, q, k, q_weight, k_weight, cos, sin, eps):
        q, k = q.contiguous(), k.contiguous()
        qw, kw = q_weight.contiguous().view(-1), k_weight.contiguous().view(-1)
        cos, sin = cos.contiguous(), sin.contiguous()
        _check(q, qw, cos, sin, eps)   # dtype / device / shape rules of the single-tensor op, both tensors
        _check(k, kw, cos, sin, eps)
        ctx.save_for_backward(q, k, qw, kw, cos, sin)
        ctx.eps = eps
        ctx.shapes = (q_weight.shape, k_weight.shape)
        ctx.pair = q.shape[:2] == k.shape[:2] and q.shape[-1] == k.shape[-1] and \
            _ops.norm_rope_qk_ok(q, k, q.shape[-1])
        if ctx.pair:
            return _ops.norm_rope_qk_fwd(q, k, qw, kw, cos, sin, eps)
        return _ops.norm_rope_fwd(q, qw, cos, sin, eps), _ops.norm_rope_fwd(k, kw, cos, sin, eps)

    @staticmethod
    def backward(ctx, grad_q, grad_k):
        q, k, qw, kw, cos, sin = ctx.saved_tensors
        if ctx.pair and grad_q is not None and grad_k is not None:
            dq, dk, dqw, dkw = _ops.norm_rope_qk_bwd(q, k, qw, kw, cos, sin, grad_q.contiguous(),
                                                     grad_k.contiguous(), ctx.eps)
            return dq, dk, dqw.view(ctx.shapes[0]), dkw.view(ctx.shapes[1]), None, None, None
        dq = dk = dqw = dkw = None
        if grad_q is not None:
            dq, dqw = _ops.norm_rope_bwd(q, qw, cos, sin, grad_q.contiguous(), ctx.eps)
            dqw = dqw.view(ctx.shapes[0])
        if grad_k is not None:
            dk, dkw = _ops.norm_rope_bwd(k, kw, cos, sin, grad_k.contiguous(), ctx.eps)
            dkw = dkw.view(ctx.shapes[1])
        return dq, dk, dqw, dkw, None, None, None


def norm_rope_pair(q, k, q_weight, k_weight, cos, sin, eps=1e-6):
    """(norm_rope(q, q_weight, ..), norm_rope(k, k_weight, ..)) with both tensors in one launch."""
    return _NormRoPEPair.apply(q, k, q_weight, k_weight, cos, sin, eps)
