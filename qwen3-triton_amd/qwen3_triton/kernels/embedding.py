"""Embedding gather with a deterministic scatter-sum backward.

Mirrors ``qwen3_triton/kernels/embedding.py:49-81``.  The reference asserts on the device for an
out-of-range id; here the kernel zeroes the row and raises a device flag that the wrapper checks
(outside graph capture), raising ValueError.
"""
import torch

from . import _ops


class _Embedding(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ids, weight):
        if not ids.is_cuda or not weight.is_cuda or ids.device != weight.device:
            raise ValueError('Same-device ROCm inputs required; no fallback')
        if ids.dtype not in (torch.int32, torch.int64) or \
                weight.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise TypeError('Integer IDs and floating point weight required')
        if not ids.is_contiguous() or not weight.is_contiguous() or weight.ndim != 2 or ids.numel() < 1:
            raise ValueError('Contiguous nonempty IDs and matrix weight required')
        if min(weight.shape) < 1:
            raise ValueError('Nonempty vocabulary and hidden dimension required')
        capturing = torch.cuda.is_current_stream_capturing()
        bad = None if capturing else torch.zeros((), dtype=torch.int32, device=ids.device)
        y = _ops.embedding_fwd(ids, weight, bad)
        if bad is not None and bool(bad.item()):
            raise ValueError('embedding ID out of range')
        ctx.save_for_backward(ids)
        ctx.weight_shape = weight.shape
        ctx.weight_dtype = weight.dtype
        return y

    @staticmethod
    def backward(ctx, dy):
        ids, = ctx.saved_tensors
        v, _ = ctx.weight_shape
        return None, _ops.embedding_bwd(ids, dy.contiguous(), v, ctx.weight_dtype)


def embedding(ids, weight):
    return _Embedding.apply(ids, weight)
