"""RMSNorm with a deterministic weight-gradient reduction.

Mirrors ``qwen3_triton/kernels/norm.py:39-66`` (``_RMSNorm`` / ``rms_norm``): same signature,
same validation, fp32 internals; the forward is ``q3_rmsnorm_fwd`` and the backward
``q3_rmsnorm_bwd`` (dx plus a fixed-order two-level dW sum, no float atomics).
"""
import torch

from . import _ops


def _validate(x, weight, eps, max_h):
    if not x.is_cuda or x.device != weight.device or x.dtype != weight.dtype:
        raise ValueError('Same-device/dtype ROCm input and weight required; no fallback')
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError('Floating point required')
    if weight.ndim != 1 or not x.is_contiguous() or not weight.is_contiguous() or \
            x.shape[-1] != weight.numel() or x.numel() < 1:
        raise ValueError('Contiguous [...,H] input and [H] weight required')
    if weight.numel() > max_h or eps <= 0:
        raise ValueError(f'Supported H<={max_h} and positive epsilon required')


class _RMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, eps, optimized):
        _validate(x, weight, eps, 8192)
        ctx.save_for_backward(x, weight)
        ctx.eps = eps
        return _ops.rmsnorm_fwd(x, weight, eps)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dx, dw = _ops.rmsnorm_bwd(x, w, dy.contiguous(), ctx.eps)
        return dx, dw, None, None


def rms_norm(x, weight, eps=1e-6, *, optimized=False):
    """``kernels/norm.py:65``."""
    return _RMSNorm.apply(x, weight, eps, optimized)


class _RMSNormFork(torch.autograd.Function):
    """The input of a residual block, x -> (x, rms_norm(x)), as one node: the residual branch's
    gradient and the norm's input gradient of x are summed inside the backward kernel
    (``q3_rmsnorm_bwd_add``) instead of by autograd with a separate add.  Same math as
    ``rms_norm`` on the second output; the first is a view of x."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        _validate(x, weight, eps, 1 << 20)   # the widest row the kernels take
        ctx.save_for_backward(x, weight)
        ctx.eps = eps
        return x.view_as(x), _ops.rmsnorm_fwd(x, weight, eps)

    @staticmethod
    def backward(ctx, dres, dy):
        x, w = ctx.saved_tensors
        if dy is None:
            return dres, None, None
        if dres is None:
            dx, dw = _ops.rmsnorm_bwd(x, w, dy.contiguous(), ctx.eps)
        else:
            dx, dw = _ops.rmsnorm_bwd_add(x, w, dy.contiguous(), dres.contiguous(), ctx.eps)
        return dx, dw, None


def rms_norm_fork(x, weight, eps=1e-6):
    """(x, rms_norm(x, weight, eps)) for a residual block ``x + f(rms_norm(x))``."""
    return _RMSNormFork.apply(x, weight, eps)
