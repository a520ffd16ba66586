"""SwiGLU silu(gate)*up, forward and backward (``qwen3_triton/kernels/activation.py:22-36``)."""
import torch

from . import _ops


class _SwiGLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, g, u):
        if not g.is_cuda or g.device != u.device or g.shape != u.shape or g.dtype != u.dtype or \
                not g.is_contiguous() or not u.is_contiguous() or g.numel() < 1:
            raise ValueError('Matching contiguous nonempty ROCm inputs required')
        if g.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise TypeError('Floating point required')
        ctx.save_for_backward(g, u)
        return _ops.swiglu_fwd(g, u)

    @staticmethod
    def backward(ctx, dy):
        g, u = ctx.saved_tensors
        return _ops.swiglu_bwd(g, u, dy.contiguous())


def swiglu(gate, up):
    return _SwiGLU.apply(gate, up)
