"""``ops/triton/attention.py:136-292``: standalone causal attention entry points on HIP kernels."""
from __future__ import annotations

import math

import torch

from qwen3_triton.kernels import _ops


def _validate(q, k, v, is_causal):
    """The checks of ``ops/triton/attention.py:151-178``, in order; then the shared dtype this build
    needs (the reference's kernel would fail to compile a mixed-dtype dot product)."""
    if not all(t.is_cuda for t in (q, k, v)):
        raise ValueError("attention_triton requires ROCm tensors")
    if not (q.ndim == k.ndim == v.ndim == 4):
        raise ValueError("q, k, and v must be rank-4 tensors")
    batch, q_heads, q_len, head_dim = q.shape
    k_batch, kv_heads, k_len, k_dim = k.shape
    if (k_batch, k_len, k_dim) != (batch, q_len, head_dim):
        raise ValueError("first kernel requires q/k sequence and head_dim shapes to match")
    if v.shape != (batch, kv_heads, q_len, head_dim):
        raise ValueError("v must have shape [batch, kv_heads, seq_len, head_dim]")
    if q_heads % kv_heads != 0:
        raise ValueError("q_heads must be divisible by kv_heads for GQA")
    if not is_causal:
        raise NotImplementedError("first attention kernel only supports causal attention")
    if head_dim <= 0 or head_dim % 2 != 0:
        raise ValueError("head_dim must be a positive even number")
    if head_dim > 256:
        raise ValueError("first attention kernel supports head_dim <= 256")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise TypeError("q, k, v must share a dtype")


def attention_triton(q, k, v, *, is_causal=True, scale=None, return_lse=False):
    """Forward causal attention for [B, H, S, D] tensors; GQA maps query heads to KV heads."""
    _validate(q, k, v, is_causal)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    out, lse = _ops.attention_fwd(q, k, v, scale)
    return (out, lse) if return_lse else out


def attention_triton_qwen_prefill(q, k, v, *, scale=None, return_lse=False):
    """Qwen prefill entry point (head_dim 128, equal query/KV lengths)."""
    if q.ndim != 4 or q.shape[-1] != 128:
        raise ValueError("Qwen prefill requires q with shape [B, Hq, S, 128]")
    if k.shape[-1] != 128 or v.shape != k.shape:
        raise ValueError("Qwen prefill requires k/v with shape [B, Hkv, S, 128]")
    if q.shape[2] != k.shape[2]:
        raise ValueError("prefill requires equal query and KV sequence lengths")
    return attention_triton(q, k, v, scale=scale, return_lse=return_lse)


def attention_triton_with_lse(q, k, v, *, is_causal=True, scale=None):
    """Forward output plus the compact LSE needed by backward."""
    return attention_triton(q, k, v, is_causal=is_causal, scale=scale, return_lse=True)


class _AttentionFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, scale):
        out, lse = attention_triton_with_lse(q, k, v, scale=scale)
        ctx.save_for_backward(q.contiguous(), k.contiguous(), v.contiguous(), out, lse)
        ctx.scale = scale
        return out

    @staticmethod
    def backward(ctx, grad_output):
        q, k, v, out, lse = ctx.saved_tensors
        return (*_ops.attention_bwd(q, k, v, out, lse, grad_output.contiguous(), ctx.scale), None)


def attention_triton_autograd(q, k, v, *, scale=None):
    """Trainable causal attention using the saved-LSE backward."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    return _AttentionFunction.apply(q, k, v, scale)
