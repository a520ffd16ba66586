"""``ops/triton/fused_qk_norm_rope.py:237-273``: fused Q/K RMSNorm + RoPE, q/k [B,S,H,D]."""
import torch

from qwen3_triton.kernels import _ops


def _check(x, w, cos, sin):
    if not x.is_cuda:
        raise ValueError("fused_qk_norm_rope requires ROCm tensors")
    if x.ndim != 4 or w.numel() != x.shape[-1] or cos.shape != (x.shape[0], x.shape[1], x.shape[3]) or \
            sin.shape != cos.shape or x.shape[-1] % 2:
        raise ValueError("expected x=[B,S,H,D], weight=[D], cos/sin=[B,S,D] with even D")
    if w.dtype != x.dtype or cos.dtype != x.dtype or sin.dtype != x.dtype:
        raise TypeError("weight and cos/sin must have the dtype of x")


class _FusedQKNormRoPEFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, q_weight, k_weight, cos, sin, eps):
        for x, w in ((q, q_weight), (k, k_weight)):
            _check(x, w, cos, sin)
        q, k = q.contiguous(), k.contiguous()
        qw, kw = q_weight.contiguous().view(-1), k_weight.contiguous().view(-1)
        cos, sin = cos.contiguous(), sin.contiguous()
        ctx.save_for_backward(q, k, qw, kw, cos, sin)
        ctx.eps = eps
        ctx.shapes = (q_weight.shape, k_weight.shape)
        return _ops.norm_rope_fwd(q, qw, cos, sin, eps), _ops.norm_rope_fwd(k, kw, cos, sin, eps)

    @staticmethod
    def backward(ctx, grad_q, grad_k):
        q, k, qw, kw, cos, sin = ctx.saved_tensors
        dq = dk = dqw = dkw = None
        if grad_q is not None:
            dq, dqw = _ops.norm_rope_bwd(q, qw, cos, sin, grad_q.contiguous(), ctx.eps)
            dqw = dqw.view(ctx.shapes[0])
        if grad_k is not None:
            dk, dkw = _ops.norm_rope_bwd(k, kw, cos, sin, grad_k.contiguous(), ctx.eps)
            dkw = dkw.view(ctx.shapes[1])
        return dq, dk, dqw, dkw, None, None, None


def fused_qk_norm_rope_triton(q, k, q_weight, k_weight, cos, sin, eps=1e-6):
    """Fused Q/K RMSNorm + RoPE, one HIP launch per tensor."""
    return _FusedQKNormRoPEFunction.apply(q, k, q_weight, k_weight, cos, sin, eps)
