"""Bias-free Linear with matrix-core forward, dX and dW GEMMs.

Mirrors ``qwen3_triton/kernels/linear.py:45-105``: ``matmul(a, b, *, optimized, output_dtype)``
computes A[M,K] @ B[K,N] for strided matrices into a contiguous result with fp32 accumulation,
and ``linear(x, weight)`` is Y = X W^T with dX = dY W and dW = dY^T X.

Dispatch: bf16/fp16 operands go to ``q3_gemm_nt`` (MFMA), which wants both operands with K
contiguous; an operand that is K-major only as a transposed view is first re-laid out by
``q3_transpose`` (a bandwidth-bound copy).  fp32 or oddly strided operands use the SIMT
``q3_gemm_strided`` kernel.  ``optimized`` is accepted for signature compatibility; the tile
plan is fixed for gfx950.
"""
import ctypes

import torch

from .. import _hip as H
from . import _ops


def _k_major_rows(t):
    """Return (tensor, row_stride) with t's rows (dim 0) K-contiguous, or None if impossible."""
    if t.stride(1) == 1 and t.stride(0) >= t.shape[1]:
        return t, t.stride(0)
    if t.stride(0) == 1 and t.stride(1) >= t.shape[0]:
        # t is the transpose of a row-major [K, rows] matrix: re-lay it out.
        src = t.t()
        if not src.is_contiguous():
            src = src.contiguous()
        tt = _ops.transpose_last2(src)
        return tt, tt.stride(0)
    return None


def _aligned(t, ld):
    return t.data_ptr() % 16 == 0 and ld % 8 == 0


def gemm_nt_into(a, lda, bnk, ldb, out, m, n, k, *, alpha=1.0, accumulate=False):
    """out[m,n] (+)= alpha * a[m,k] . bnk[n,k]^T on the matrix cores (a, bnk K-contiguous rows)."""
    H.call("q3_gemm_nt", H.code(a.dtype), H.code(out.dtype), a.data_ptr(), lda, bnk.data_ptr(), ldb,
           out.data_ptr(), out.stride(0), m, n, k, float(alpha), int(accumulate), H.stream())


def gate_up_swiglu_into(x, wg, wu, g, u, y, m, n, k):
    """g = x wg^T, u = x wu^T, y = silu(g) * u in one matrix-core GEMM (M % 256 == 0, N % 128 == 0,
    K % 64 == 0; contiguous [M, K] x and [N, K] weights, contiguous [M, N] outputs); g and u None:
    y only."""
    H.call("q3_gemm_gate_up_swiglu", H.code(x.dtype), x.data_ptr(), k, wg.data_ptr(), wu.data_ptr(), k,
           None if g is None else g.data_ptr(), None if u is None else u.data_ptr(), y.data_ptr(), n, m, n, k,
           H.stream())


def gate_up_swiglu_t_into(x, wg, wu, g, u, y, yt, m, n, k):
    """``gate_up_swiglu_into`` that also writes yt = y^T [n, m] (the down projection's weight-gradient
    operand) from the same epilogue."""
    H.call("q3_gemm_gate_up_swiglu_t", H.code(x.dtype), x.data_ptr(), k, wg.data_ptr(), wu.data_ptr(), k,
           g.data_ptr(), u.data_ptr(), y.data_ptr(), n, yt.data_ptr(), yt.stride(0), m, n, k, H.stream())


def gemm_nt_residual_into(a, lda, bnk, ldb, res, out, m, n, k):
    """out[m, n] = res + a[m, k] . bnk[n, k]^T (the GEMM output rounded, then the residual added and
    rounded again).  One matrix-core launch, bit-identical to the GEMM followed by the add kernel;
    shapes whose 256 x 256 grid would leave half of the CUs idle and whose K is long (the 2048-token
    prefill's down projection) run as two K halves into an fp32 workspace and one combining pass instead."""
    ws_bytes = H.query("q3_gemm_nt_residual_workspace_bytes", m, n, k)
    ws = H.workspace(ws_bytes, a.device) if ws_bytes else None
    H.call("q3_gemm_nt_residual_ws", H.code(a.dtype), a.data_ptr(), lda, bnk.data_ptr(), ldb, res.data_ptr(),
           res.stride(0), out.data_ptr(), out.stride(0), m, n, k, None if ws is None else ws.data_ptr(),
           ws_bytes, H.stream())


def gemm_nt_residual_norm_into(a, lda, bnk, ldb, res, out, norm_w, eps, y, m, n, k):
    """``gemm_nt_residual_into`` that also writes y = rms_norm(out, norm_w, eps) (the next block's
    normed input; N <= 8192): in the same combining pass on the two-K-halves plan, else a separate
    norm launch."""
    ws_bytes = H.query("q3_gemm_nt_residual_workspace_bytes", m, n, k)
    ws = H.workspace(ws_bytes, a.device) if ws_bytes else None
    H.call("q3_gemm_nt_residual_norm_ws", H.code(a.dtype), a.data_ptr(), lda, bnk.data_ptr(), ldb, res.data_ptr(),
           res.stride(0), out.data_ptr(), out.stride(0), norm_w.data_ptr(), float(eps), y.data_ptr(), y.stride(0),
           m, n, k, None if ws is None else ws.data_ptr(), ws_bytes, H.stream())


def gemm_residual_ok(dtype, m, n, k):
    """The fused residual epilogue serves 16-bit data in full 128 x 128 (or 256 x 256) tiles."""
    return dtype in (torch.bfloat16, torch.float16) and m % 128 == 0 and n % 128 == 0 and k % 64 == 0


def swiglu_bwd_gemm_into(dy, wt, g, u, dg, du, dgt, dut, m, n, k):
    """dg, du (and their transposes dgt, dut when given) of y = silu(g) * u for the upstream gradient
    dY = dy wt^T, computed in one matrix-core GEMM whose epilogue runs the SwiGLU backward
    (dy [m, k], wt [n, k]; g, u, dg, du [m, n] views at a common row stride; M % 256 == 0,
    N % 256 == 0, K % 64 == 0)."""
    H.call("q3_gemm_swiglu_bwd", H.code(dy.dtype), dy.data_ptr(), dy.stride(0), wt.data_ptr(), wt.stride(0),
           g.data_ptr(), u.data_ptr(), g.stride(0), dg.data_ptr(), du.data_ptr(), dg.stride(0),
           0 if dgt is None else dgt.data_ptr(), 0 if dut is None else dut.data_ptr(),
           0 if dgt is None else dgt.stride(0), m, n, k, H.stream())


def swiglu_bwd_gemm_ok(dtype, m, n, k):
    return dtype in (torch.bfloat16, torch.float16) and m % 256 == 0 and n % 256 == 0 and k % 64 == 0


def gemm_nt_multi_into(a, weights, outs, m, k):
    """outs[i][m, n_i] = a[m, k] . weights[i][n_i, k]^T for up to 3 weights in one matrix-core launch
    (contiguous a / weights / outs; M % 256 == 0, each n_i % 256 == 0, K % 64 == 0)."""
    n = len(weights)
    bs = (ctypes.c_void_p * n)(*[w.data_ptr() for w in weights])
    cs = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    ns = (ctypes.c_int64 * n)(*[w.shape[0] for w in weights])
    lds = (ctypes.c_int64 * n)(*[o.stride(0) for o in outs])
    H.call("q3_gemm_nt_multi", H.code(a.dtype), a.data_ptr(), k, n, bs, k, cs, ns, lds, m, k, H.stream())


def gemm_multi_ok(x, m, k, weights):
    """The one-launch path needs 16-bit data and full 128 x 128 (or 256 x 256) tiles."""
    return x.dtype in (torch.bfloat16, torch.float16) and len(weights) <= 3 and m % 128 == 0 and k % 64 == 0 and \
        all(w.shape[0] % 128 == 0 for w in weights)


def gate_up_fused_ok(x, m, n, k):
    return x.dtype in (torch.bfloat16, torch.float16) and m % 256 == 0 and n % 128 == 0 and k % 64 == 0


def matmul_into(a, b, out, *, alpha=1.0, accumulate=False):
    m, k = a.shape
    n = b.shape[1]
    if a.dtype in (torch.bfloat16, torch.float16) and k % 8 == 0:
        ar = _k_major_rows(a)
        br = _k_major_rows(b.t())
        if ar is not None and br is not None and _aligned(*ar) and _aligned(*br):
            gemm_nt_into(ar[0], ar[1], br[0], br[1], out, m, n, k, alpha=alpha, accumulate=accumulate)
            return out
    H.call("q3_gemm_strided", H.code(a.dtype), H.code(out.dtype), a.data_ptr(), a.stride(0), a.stride(1),
           b.data_ptr(), b.stride(0), b.stride(1), out.data_ptr(), out.stride(0), m, n, k, float(alpha),
           int(accumulate), H.stream())
    return out


def matmul(a, b, *, optimized=False, output_dtype=None):
    """A[M,K] @ B[K,N]; strided matrices, contiguous result, FP32 accumulation."""
    if not (a.is_cuda and b.is_cuda) or a.device != b.device:
        raise ValueError('Same-device ROCm matrices required; no fallback')
    if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[0]:
        raise ValueError('Expected [M,K] and [K,N]')
    if a.dtype != b.dtype or a.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError('Matching BF16/FP16/FP32 matrices required')
    if min(*a.shape, *b.shape) < 1 or min(*a.stride(), *b.stride()) < 1:
        raise ValueError('Nonempty, positive-stride matrices required')
    dtype = output_dtype or a.dtype
    if dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError('Floating point output required')
    out = torch.empty((a.shape[0], b.shape[1]), device=a.device, dtype=dtype)
    return matmul_into(a, b, out)


class _Linear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, optimized):
        if x.ndim < 2 or weight.ndim != 2 or x.shape[-1] != weight.shape[1]:
            raise ValueError('Expected X[...,K] and weight[N,K]')
        if not x.is_contiguous():
            raise ValueError('Linear input must be contiguous; no hidden layout copy')
        flat = x.view(-1, x.shape[-1])
        y = matmul(flat, weight.t(), optimized=optimized)
        ctx.save_for_backward(flat, weight)
        ctx.shape = x.shape
        ctx.optimized = optimized
        return y.view(*x.shape[:-1], weight.shape[0])

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dy = dy.contiguous().view(-1, w.shape[0])
        dx = matmul(dy, w, optimized=ctx.optimized).view(ctx.shape) if ctx.needs_input_grad[0] else None
        dw = matmul(dy.t(), x, optimized=ctx.optimized) if ctx.needs_input_grad[1] else None
        return dx, dw, None


def linear(x, weight, *, optimized=False):
    """``kernels/linear.py:104``."""
    return _Linear.apply(x, weight, optimized)


class _LinearResidual(torch.autograd.Function):
    """res + X W^T (an output projection and the residual sum after it) as one op: one matrix-core
    launch with the residual in the epilogue where the shape allows it; backward dX = dY W,
    dW = dY^T X, dRes = dY."""

    @staticmethod
    def forward(ctx, x, weight, res, optimized):
        if x.ndim < 2 or weight.ndim != 2 or x.shape[-1] != weight.shape[1]:
            raise ValueError('Expected X[...,K] and weight[N,K]')
        if not x.is_contiguous() or not res.is_contiguous():
            raise ValueError('Linear input and residual must be contiguous; no hidden layout copy')
        if res.shape != (*x.shape[:-1], weight.shape[0]) or res.dtype != x.dtype or res.device != x.device:
            raise ValueError('residual must match the projection output')
        flat = x.view(-1, x.shape[-1])
        m, k = flat.shape
        n = weight.shape[0]
        if gemm_residual_ok(x.dtype, m, n, k) and weight.dtype == x.dtype and weight.is_contiguous():
            out = torch.empty((m, n), device=x.device, dtype=x.dtype)
            gemm_nt_residual_into(flat, k, weight, k, res.view(m, n), out, m, n, k)
        else:
            out = _ops.add(res.view(m, n), matmul(flat, weight.t(), optimized=optimized))
        ctx.save_for_backward(flat, weight)
        ctx.shape = x.shape
        ctx.optimized = optimized
        return out.view(res.shape)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dyf = dy.contiguous().view(-1, w.shape[0])
        dx = matmul(dyf, w, optimized=ctx.optimized).view(ctx.shape) if ctx.needs_input_grad[0] else None
        dw = matmul(dyf.t(), x, optimized=ctx.optimized) if ctx.needs_input_grad[1] else None
        return dx, dw, dy, None


def linear_residual(x, weight, res, *, optimized=False):
    """``res + linear(x, weight)`` (``kernels/residual.py:30`` after ``kernels/linear.py:104``)."""
    return _LinearResidual.apply(x, weight, res, optimized)


class _SharedInputProjections(torch.autograd.Function):
    """Y_i = X W_i^T for several weights sharing one input (the q/k/v projections).  Forward runs
    one GEMM per weight; backward packs the output gradients side by side, so dX = [dY_0 | dY_1 | ...]
    [W_0; W_1; ...] is a single matrix-core GEMM (one rounding, no partial sums added afterwards), X is
    transposed once, and one GEMM produces every weight gradient as a row block."""

    @staticmethod
    def forward(ctx, x, *weights):
        flat = x.view(-1, x.shape[-1])
        m, k = flat.shape
        if gemm_multi_ok(x, m, k, weights):
            # one launch over the weights side by side (the narrow K / V projections alone would leave
            # half of the CUs idle)
            outs = [torch.empty((m, w.shape[0]), device=x.device, dtype=x.dtype) for w in weights]
            gemm_nt_multi_into(flat, weights, outs, m, k)
            outs = [o.view(*x.shape[:-1], o.shape[1]) for o in outs]
        else:
            outs = [matmul(flat, w.t()).view(*x.shape[:-1], w.shape[0]) for w in weights]
        ctx.save_for_backward(flat, *weights)
        ctx.shape = x.shape
        return tuple(outs)

    @staticmethod
    def backward(ctx, *grads):
        flat, *weights = ctx.saved_tensors
        m, k = flat.shape
        ns = [w.shape[0] for w in weights]
        nt = sum(ns)
        dev, dt = flat.device, flat.dtype
        dcat = torch.empty((m, nt), device=dev, dtype=dt)
        wt = torch.empty((k, nt), device=dev, dtype=dt)
        col = 0
        for gr, w, n in zip(grads, weights, ns):
            blk = dcat[:, col:col + n]
            if gr is None:
                blk.zero_()
            else:
                _ops.copy_into(gr.contiguous().view(m, n), blk)
            _ops.transpose_into(w, wt[:, col:col + n])
            col += n
        dx = torch.empty((m, k), device=dev, dtype=dt)
        gemm_nt_into(dcat, nt, wt, nt, dx, m, k, nt)
        dct = _ops.transpose_into(dcat, torch.empty((nt, m), device=dev, dtype=dt))
        xt = _ops.transpose_into(flat, torch.empty((k, m), device=dev, dtype=dt))
        dw = torch.empty((nt, k), device=dev, dtype=dt)
        gemm_nt_into(dct, m, xt, m, dw, nt, k, m)
        dws, row = [], 0
        for n in ns:
            dws.append(dw[row:row + n])
            row += n
        return (dx.view(ctx.shape), *dws)


def shared_input_projections(x, weights, *, optimized=False):
    """[X W_i^T for W_i in weights]; the fused backward needs 16-bit contiguous operands with every
    dimension a multiple of 8, otherwise each projection is an ordinary ``linear``."""
    ok = x.dtype in (torch.bfloat16, torch.float16) and x.is_contiguous() and x.shape[-1] % 8 == 0 and \
        (x.numel() // x.shape[-1]) % 8 == 0 and \
        all(w.dtype == x.dtype and w.is_contiguous() and w.ndim == 2 and w.shape[1] == x.shape[-1] and
            w.shape[0] % 8 == 0 for w in weights)
    if not ok:
        return [linear(x, w, optimized=optimized) for w in weights]
    return list(_SharedInputProjections.apply(x, *weights))

