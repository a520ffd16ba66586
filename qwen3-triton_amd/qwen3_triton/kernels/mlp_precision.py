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
from .linear import (gate_up_fused_ok, gate_up_swiglu_into, gate_up_swiglu_t_into, gemm_nt_into, gemm_nt_residual_into, gemm_residual_ok,
                     linear, linear_residual, matmul, matmul_into, swiglu_bwd_gemm_into, swiglu_bwd_gemm_ok)


def _check(x, wg, wu):
    if not x.is_cuda or x.ndim < 2 or wg.ndim != 2 or wg.shape != wu.shape or x.shape[-1] != wg.shape[1]:
        raise ValueError('Expected ROCm X[...,K] and matching [N,K] gate/up weights')
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16) or \
            any(t.device != x.device or t.dtype != x.dtype or not t.is_contiguous() for t in (x, wg, wu)):
        raise ValueError('Matching contiguous floating point ROCm inputs required')
    m, k, n = x.numel() // x.shape[-1], x.shape[-1], wg.shape[0]
    if min(m, k, n) < 1:
        raise ValueError('Nonempty inputs required')
    return m, k, n


def _gate_up_y(x, wg, wu):
    """Y alone (no autograd: nothing is saved, so the fused GEMM skips the G and U stores)."""
    m, k, n = _check(x, wg, wu)
    flat = x.view(m, k)
    if gate_up_fused_ok(x, m, n, k):
        y = torch.empty((m, n), device=x.device, dtype=x.dtype)
        gate_up_swiglu_into(flat, wg, wu, None, None, y, m, n, k)
    else:
        y = _ops.swiglu_fwd(matmul(flat, wg.t()), matmul(flat, wu.t()))
    return y.view(*x.shape[:-1], n)


class _GateUp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, wg, wu, optimized):
        m, k, n = _check(x, wg, wu)
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
    """``kernels/mlp_precision.py:65``.  Without autograd (inference, or no input needing a gradient)
    only Y is formed: the same values, without the G and U the backward would need."""
    if not (torch.is_grad_enabled() and any(t.requires_grad for t in (x, gate_weight, up_weight))):
        return _gate_up_y(x, gate_weight, up_weight)
    return _GateUp.apply(x, gate_weight, up_weight, optimized)


def _gate_up_forward(flat, wg, wu, m, n, k):
    if gate_up_fused_ok(flat, m, n, k):
        g, u, y = (torch.empty((m, n), device=flat.device, dtype=flat.dtype) for _ in range(3))
        gate_up_swiglu_into(flat, wg, wu, g, u, y, m, n, k)
        return g, u, y
    g = matmul(flat, wg.t())
    u = matmul(flat, wu.t())
    return g, u, _ops.swiglu_fwd(g, u)


class _MLPBlock(torch.autograd.Function):
    """out = (silu(X Wg^T) * (X Wu^T)) Wd^T as one op, so the backward can run the SwiGLU backward in
    the epilogue of the down projection's input-gradient GEMM: dY never reaches memory, and the same
    epilogue writes [dG | dU] row-major (the gate/up dX GEMM operand) and transposed (the gate/up
    weight-gradient GEMM operand), replacing the SwiGLU backward kernel and one transpose pass.
    Every GEMM and rounding point is the one of ``gate_up_swiglu`` followed by ``linear``."""

    @staticmethod
    def forward(ctx, x, wg, wu, wd, res):
        m, k, n = x.numel() // x.shape[-1], x.shape[-1], wg.shape[0]
        h = wd.shape[0]
        flat = x.view(m, k)
        yt = None
        if gate_up_fused_ok(flat, m, n, k):
            # the epilogue also stores Y^T, the down weight-gradient operand of the backward
            g, u, y = (torch.empty((m, n), device=x.device, dtype=x.dtype) for _ in range(3))
            yt = torch.empty((n, m), device=x.device, dtype=x.dtype)
            gate_up_swiglu_t_into(flat, wg, wu, g, u, y, yt, m, n, k)
        else:
            g, u, y = _gate_up_forward(flat, wg, wu, m, n, k)
        out = torch.empty((m, h), device=x.device, dtype=x.dtype)
        if res is None:
            gemm_nt_into(y, n, wd, n, out, m, h, n)
        elif gemm_residual_ok(x.dtype, m, h, n):  # the residual sum rides in the down GEMM's epilogue
            gemm_nt_residual_into(y, n, wd, n, res.view(m, h), out, m, h, n)
        else:
            gemm_nt_into(y, n, wd, n, out, m, h, n)
            out = _ops.add(res.view(m, h), out)
        ctx.save_for_backward(x, wg, wu, wd, g, u, y if yt is None else yt)
        ctx.has_yt = yt is not None
        ctx.has_res = res is not None
        return out.view(*x.shape[:-1], h)

    @staticmethod
    def backward(ctx, dout):
        x, wg, wu, wd, g, u, yy = ctx.saved_tensors
        m, k, n = x.numel() // x.shape[-1], x.shape[-1], wg.shape[0]
        h = wd.shape[0]
        dev, dt = x.device, x.dtype
        dof = dout.contiguous().view(m, h)
        if ctx.has_yt:  # dWd = dOut^T Y with Y^T stored by the forward epilogue
            dwd = torch.empty((h, n), device=dev, dtype=dt)
            doft = _ops.transpose_into(dof, torch.empty((h, m), device=dev, dtype=dt))
            gemm_nt_into(doft, m, yy, m, dwd, h, n, m)
        else:
            dwd = matmul(dof.t(), yy)
        wdt = _ops.transpose_into(wd, torch.empty((n, h), device=dev, dtype=dt))
        dgu = torch.empty((m, 2 * n), device=dev, dtype=dt)
        dgut = torch.empty((2 * n, m), device=dev, dtype=dt)
        swiglu_bwd_gemm_into(dof, wdt, g, u, dgu[:, :n], dgu[:, n:], dgut[:n], dgut[n:], m, n, h)
        wt = torch.empty((k, 2 * n), device=dev, dtype=dt)
        _ops.transpose_into(wg, wt[:, :n])
        _ops.transpose_into(wu, wt[:, n:])
        dx = torch.empty((m, k), device=dev, dtype=dt)
        gemm_nt_into(dgu, 2 * n, wt, 2 * n, dx, m, k, 2 * n)
        xt = _ops.transpose_into(x.view(m, k), torch.empty((k, m), device=dev, dtype=dt))
        dw = torch.empty((2 * n, k), device=dev, dtype=dt)
        gemm_nt_into(dgut, m, xt, m, dw, 2 * n, k, m)
        return dx.view(x.shape), dw[:n], dw[n:], dwd, (dout if ctx.has_res else None)


def mlp_block(x, gate_weight, up_weight, down_weight, *, optimized=False, residual=None):
    """down(silu(gate(x)) * up(x)) (+ ``residual``) -- ``components.py`` MLP: ``gate_up_swiglu`` then the
    down ``linear`` (then the residual sum) -- with the fused backward above when every operand suits
    the matrix-core epilogue (16-bit contiguous operands, tokens and intermediate size multiples of
    256, hidden a multiple of 64); otherwise exactly that composition."""
    m, k, n = x.numel() // x.shape[-1], x.shape[-1], gate_weight.shape[0]
    ok = x.is_cuda and x.is_contiguous() and down_weight.ndim == 2 and down_weight.shape[1] == n and \
        gate_weight.shape == up_weight.shape and gate_weight.shape[1] == k and \
        all(t.dtype == x.dtype and t.device == x.device and t.is_contiguous()
            for t in (gate_weight, up_weight, down_weight)) and \
        swiglu_bwd_gemm_ok(x.dtype, m, n, down_weight.shape[0]) and k % 8 == 0 and down_weight.shape[0] % 8 == 0
    if residual is not None:
        ok = ok and residual.is_contiguous() and residual.dtype == x.dtype and residual.device == x.device and \
            residual.shape == (*x.shape[:-1], down_weight.shape[0])
    if not ok:
        y = gate_up_swiglu(x, gate_weight, up_weight, optimized=optimized)
        if residual is None:
            return linear(y, down_weight, optimized=optimized)
        return linear_residual(y, down_weight, residual, optimized=optimized)
    return _MLPBlock.apply(x, gate_weight, up_weight, down_weight, residual)
