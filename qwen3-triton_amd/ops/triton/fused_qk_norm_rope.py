"""``ops/triton/fused_qk_norm_rope.py:237-273``: fused Q/K RMSNorm + RoPE, q/k [B,S,H,D]."""
import torch

from qwen3_triton.kernels import _ops
from qwen3_triton.kernels.norm_rope import norm_rope_pair


def _check(x, w, cos, sin):
    """The argument checks of the reference's ``_fused_one`` (``fused_qk_norm_rope.py:68-94``)."""
    if not all(t.is_cuda for t in (x, w, cos, sin)):
        raise ValueError("fused_norm_rope_triton requires ROCm tensors")
    if x.ndim != 4 or cos.ndim != 3 or sin.shape != cos.shape:
        raise ValueError("expected x=[batch,seq,heads,head_dim], cos/sin=[batch,seq,head_dim]")
    b, s, _, d = x.shape
    if cos.shape != (b, s, d):
        raise ValueError("cos/sin shape must be [batch,seq,head_dim]")
    if w.shape != (d,):
        raise ValueError("weight shape must be [head_dim]")
    if d % 2:
        raise ValueError("head_dim must be even")
    if d > 65536:
        raise ValueError("head_dim is too large for this first kernel")


class _Cast(torch.autograd.Function):
    """A dtype change on the HIP cast kernel whose gradient is cast back to the input's dtype."""

    @staticmethod
    def forward(ctx, x, dtype):
        ctx.dtype = x.dtype
        return _ops.cast(x.contiguous(), dtype)

    @staticmethod
    def backward(ctx, g):
        return _ops.cast(g.contiguous(), ctx.dtype), None


def fused_qk_norm_rope_triton(q, k, q_weight, k_weight, cos, sin, eps=1e-6):
    """Fused Q/K RMSNorm + RoPE: one HIP launch for both tensors per direction (one per tensor for
    shapes outside the vector path).  As in the reference, the rotary tables get no gradient, and
    weights or tables of another dtype than the activations are read as fp32: the op then runs in
    fp32 and its outputs (and input gradients) are stored in the activations' dtype."""
    for x, w in ((q, q_weight), (k, k_weight)):
        _check(x, w, cos, sin)
    cos, sin = cos.detach(), sin.detach()
    if all(t.dtype == q.dtype for t in (k, q_weight, k_weight, cos, sin)):
        return norm_rope_pair(q, k, q_weight, k_weight, cos, sin, eps)
    f32 = torch.float32
    yq, yk = norm_rope_pair(_Cast.apply(q, f32), _Cast.apply(k, f32), _Cast.apply(q_weight, f32),
                            _Cast.apply(k_weight, f32), _ops.cast(cos.contiguous(), f32),
                            _ops.cast(sin.contiguous(), f32), eps)
    return _Cast.apply(yq, q.dtype), _Cast.apply(yk, k.dtype)
