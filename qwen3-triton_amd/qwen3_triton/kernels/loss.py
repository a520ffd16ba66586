"""Causal token-mean cross-entropy on materialised logits.

Mirrors ``qwen3_triton/kernels/loss.py:46-71`` (``_CausalCE`` / ``causal_cross_entropy``): row
(b, s < S-1) predicts labels[b, s+1], loss = mean over non-ignored rows of lse - z_label, and the
backward writes (softmax - onehot) * up / count.  An out-of-range label raises ValueError (the
reference asserts on the device).
"""
import torch

from . import _ops


class _CausalCE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, labels, ignore_index, optimized):
        if not logits.is_cuda or logits.device != labels.device or logits.ndim != 3 or \
                labels.shape != logits.shape[:2]:
            raise ValueError('ROCm [B,S,V] logits and same-device [B,S] labels required')
        if labels.dtype != torch.int64 or not logits.is_contiguous() or not labels.is_contiguous():
            raise ValueError('Contiguous logits/int64 labels required')
        if logits.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise TypeError('Floating point logits required')
        b, s, v = logits.shape
        if b < 1 or s < 2 or v < 1:
            raise ValueError('Nonempty batch/vocabulary and at least 2 tokens required')
        tgt = _ops.ce_shift_labels(labels, ignore_index)
        st = _ops.CEState(b * s, 1, logits.device)
        st.stats(0, logits, v, v, 0, tgt)
        loss = st.finish(tgt, v, ignore_index)
        ctx.save_for_backward(logits, tgt, st.lse, st.count)
        ctx.ignore = ignore_index
        return loss.clone()

    @staticmethod
    def backward(ctx, dy):
        x, tgt, lse, count = ctx.saved_tensors
        b, s, v = x.shape
        dx = torch.empty_like(x)
        _ops.ce_grad(x, v, v, 0, tgt, lse, count, dy.float().contiguous(), dx, v, v, ctx.ignore)
        return dx, None, None, None


def causal_cross_entropy(logits, labels, *, ignore_index=-100, optimized=False):
    """``kernels/loss.py:70``."""
    return _CausalCE.apply(logits, labels, ignore_index, optimized)
