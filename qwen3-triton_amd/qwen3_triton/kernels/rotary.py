"""Split-half rotary tables and application on [B,S,H,D].

Mirrors ``qwen3_triton/kernels/rotary.py:36-66``: ``rotary_tables(position_ids, inv_freq, dtype)``
(fp32 angle = pos * inv_freq, cos/sin stored in ``dtype``) and ``apply_rotary(x, cos, sin)``
with its transpose as the backward.
"""
import torch

from . import _ops


def rotary_tables(position_ids, inv_freq, dtype):
    if not position_ids.is_cuda or inv_freq.device != position_ids.device:
        raise ValueError('Same ROCm device required')
    if position_ids.ndim != 2 or not position_ids.is_contiguous() or \
            position_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError('Contiguous integer [B,S] position IDs required')
    if inv_freq.dtype != torch.float32 or inv_freq.ndim != 1 or not inv_freq.is_contiguous():
        raise ValueError('Contiguous FP32 frequency buffer required')
    if dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError('Floating point output required')
    if position_ids.numel() < 1 or inv_freq.numel() < 1:
        raise ValueError('Nonempty positions/frequencies required')
    return _ops.rope_tables(position_ids, inv_freq, dtype)


class _Rotary(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, cos, sin):
        if x.ndim != 4 or cos.shape != sin.shape or cos.shape != (x.shape[0], x.shape[1], x.shape[3]) or \
                x.shape[-1] % 2:
            raise ValueError('Expected [B,S,H,D] and matching [B,S,D], even D')
        if not x.is_cuda or any(t.device != x.device or t.dtype != x.dtype or not t.is_contiguous()
                                for t in (x, cos, sin)):
            raise ValueError('Same-device/dtype contiguous ROCm tensors required')
        if cos.requires_grad or sin.requires_grad:
            raise ValueError('Fixed frequency buffers only')
        ctx.save_for_backward(cos, sin)
        return _ops.rope_apply(x, cos, sin, layout=0, backward=False)

    @staticmethod
    def backward(ctx, dy):
        cos, sin = ctx.saved_tensors
        return _ops.rope_apply(dy.contiguous(), cos, sin, layout=0, backward=True), None, None


def apply_rotary(x, cos, sin):
    """``kernels/rotary.py:65``."""
    return _Rotary.apply(x, cos, sin)
