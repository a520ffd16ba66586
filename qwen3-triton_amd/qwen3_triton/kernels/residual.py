"""Residual addition (``qwen3_triton/kernels/residual.py:13-30``); the derivative is an alias."""
import torch

from . import _ops


class _Residual(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b):
        if not a.is_cuda or a.device != b.device or a.shape != b.shape or a.dtype != b.dtype:
            raise ValueError('Matching same-device ROCm tensors required; no fallback')
        if not a.is_contiguous() or not b.is_contiguous() or a.numel() < 1:
            raise ValueError('Contiguous nonempty residual inputs required')
        if a.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise TypeError('Floating point inputs required')
        return _ops.add(a, b)

    @staticmethod
    def backward(ctx, dy):
        return dy, dy


def residual_add(a, b):
    return _Residual.apply(a, b)
