"""Gate/up projections + SwiGLU as one autograd op.

Mirrors ``qwen3_triton/kernels/mlp_precision.py:16-66`` (``_GateUp`` / ``gate_up_swiglu``):
forward G = X Wg^T, U = X Wu^T, Y = silu(G)*U, saving G and U; backward = SwiGLU backward,
dX = dG Wg + dU Wu (fp32 accumulation across both products, one rounding), dWg = dG^T X,
dWu = dU^T X.
"""
import torch

from . import _ops
from .linear import matmul, matmul_into


class _GateUp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, wg, wu, optimized):
        if not x.is_cuda or x.ndim < 2 or wg.ndim != 2 or wg.shape != wu.shape or x.shape[-1] != wg.shape[1]:
            raise ValueError('Expected ROCm X[...,K] and matching [N,K] gate/up weights')
        if x.dtype not in (torch.float32, torch.bfloat16, torch.float16) or \
                any(t.device != x.device or t.dtype != x.dtype or not t.is_contiguous() for t in (x, wg, wu)):
            raise ValueError('Matching contiguous floating point ROCm inputs required')
        m, k, n = x.numel() // x.shape[-1], x.shape[-1], wg.shape[0]
        if min(m, k, n) < 1:
            raise ValueError('Nonempty inputs required')
        flat = x.view(m, k)
        g = matmul(flat, wg.t())
        u = matmul(flat, wu.t())
        y = _ops.swiglu_fwd(g, u)
        ctx.save_for_backward(x, wg, wu, g, u)
        return y.view(*x.shape[:-1], n)

    @staticmethod
    def backward(ctx, dy):
        x, wg, wu, g, u = ctx.saved_tensors
        m, k, n = x.numel() // x.shape[-1], x.shape[-1], wg.shape[0]
        dg, du = _ops.swiglu_bwd(g, u, dy.contiguous().view(m, n))
        flat = x.view(m, k)
        acc = torch.empty((m, k), device=x.device, dtype=torch.float32)
        matmul_into(dg, wg, acc)
        matmul_into(du, wu, acc, accumulate=True)
        dx = _ops.cast(acc, x.dtype).view(x.shape)
        dwg = matmul(dg.t(), flat)
        dwu = matmul(du.t(), flat)
        return dx, dwg, dwu, None


def gate_up_swiglu(x, gate_weight, up_weight, *, optimized=False):
    """``kernels/mlp_precision.py:65``."""
    return _GateUp.apply(x, gate_weight, up_weight, optimized)
