"""Gate/up projections + SwiGLU as one autograd op.

Mirrors ``qwen3_triton/kernels/mlp_precision.py:16-66`` (``_GateUp`` / ``gate_up_swiglu``):
forward G = X Wg^T, U = X Wu^T, Y = silu(G)*U, saving G and U -- one matrix-core GEMM over both
weights with the SwiGLU in its epilogue (``q3_gemm_gate_up_swiglu``) when M % 256 == 0 and
N % 128 == 0, else two GEMMs and the SwiGLU kernel; backward = SwiGLU backward,
dX = dG Wg + dU Wu (fp32 accumulation across both products, one rounding), dWg = dG^T X,
dWu = dU^T X.  On the matrix cores the backward keeps dG and dU side by side in one [M, 2N]
buffer, so dX is a single GEMM over K = 2N and both weight gradients come from one GEMM.
"""
import torch

from . import _ops
from .linear import gate_up_fused_ok, gate_up_swiglu_into, gemm_nt_into, matmul, matmul_into


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
        if gate_up_fused_ok(x, m, n, k):
            # one GEMM over both weights; the SwiGLU runs in its epilogue
            g, u, y = (torch.empty((m, n), device=x.device, dtype=x.dtype) for _ in range(3))
            gate_up_swiglu_into(flat, wg, wu, g, u, y, m, n, k)
        else:
            g = matmul(flat, wg.t())
            u = matmul(flat, wu.t())
            y = _ops.swiglu_fwd(g, u)
        ctx.save_for_backward(x, wg, wu, g, u)
        return y.view(*x.shape[:-1], n)

    @staticmethod
    def backward(ctx, dy):
        x, wg, wu, g, u = ctx.saved_tensors
        m, k, n = x.numel() // x.shape[-1], x.shape[-1], wg.shape[0]
        flat = x.view(m, k)
        dyf = dy.contiguous().view(m, n)
        if x.dtype in (torch.bfloat16, torch.float16) and k % 8 == 0 and n % 8 == 0 and m % 8 == 0:
            # Gate and up side by side: [dG | dU] is one [M, 2N] operand, so dX = [dG | dU] [Wg; Wu] is one
            # matrix-core GEMM over K = 2N (one rounding, no fp32 partial), and [dWg; dWu] = [dG | dU]^T X
            # is one GEMM whose two row blocks are the weight gradients.
            dgu = torch.empty((m, 2 * n), device=x.device, dtype=x.dtype)
            _ops.swiglu_bwd_into(g.view(m, n), u.view(m, n), dyf, dgu[:, :n], dgu[:, n:])
            wt = torch.empty((k, 2 * n), device=x.device, dtype=x.dtype)
            _ops.transpose_into(wg, wt[:, :n])
            _ops.transpose_into(wu, wt[:, n:])
            dx = torch.empty((m, k), device=x.device, dtype=x.dtype)
            gemm_nt_into(dgu, 2 * n, wt, 2 * n, dx, m, k, 2 * n)
            dgut = _ops.transpose_into(dgu, torch.empty((2 * n, m), device=x.device, dtype=x.dtype))
            xt = _ops.transpose_into(flat, torch.empty((k, m), device=x.device, dtype=x.dtype))
            dw = torch.empty((2 * n, k), device=x.device, dtype=x.dtype)
            gemm_nt_into(dgut, m, xt, m, dw, 2 * n, k, m)
            return dx.view(x.shape), dw[:n], dw[n:], None
        dg, du = _ops.swiglu_bwd(g, u, dyf)
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
