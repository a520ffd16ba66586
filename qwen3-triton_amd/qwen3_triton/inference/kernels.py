"""Inference-only launchers: positions, KV-cache append, cached attention, small-M linear, greedy
select, and forward-only norms.  Mirrors ``qwen3_triton/inference/kernels.py`` (names and call
shapes); every op is a HIP kernel behind libq3hip.so.
"""
import torch

from .. import _hip as H
from ..kernels import _ops
from ..kernels.linear import matmul


def positions(batch, sequence, start, device):
    """``inference/kernels.py:18``: [B,S] int64 positions start..start+S-1."""
    return _ops.positions(batch, sequence, start, device)


def append(k, v, cache_k, cache_v, start):
    """``inference/kernels.py:33``: write k/v [B,S,Hkv,D] into the caches [B,Hkv,C,D] at ``start``."""
    b, s, h, d = k.shape
    H.call("q3_kv_append", H.code(k.dtype), k.data_ptr(), v.data_ptr(), cache_k.data_ptr(), cache_v.data_ptr(), b, s,
           h, d, cache_k.shape[2], start, H.stream())


def attention(q, cache_k, cache_v, start, *, split_decode=False):
    """``inference/kernels.py:95``: q [B,S,Hq,D] against cache positions [0, start+S).

    S == 1 runs the split-KV decode kernel; S > 1 (prefill, chunked prefill) runs the flash kernel
    on the cache in place (the query block is the suffix of the key range)."""
    b, s, hq, d = q.shape
    hkv = cache_k.shape[1]
    total = start + s
    if s == 1 and d == 128 and q.dtype in (torch.bfloat16, torch.float16):
        out = torch.empty_like(q)
        ws = H.workspace(H.query("q3_decode_attention_workspace_bytes", b, hq, total), q.device)
        H.call("q3_decode_attention", H.code(q.dtype), q.data_ptr(), q.stride(0), q.stride(2), cache_k.data_ptr(),
               cache_v.data_ptr(), cache_k.stride(0), cache_k.stride(1), out.data_ptr(), out.stride(0),
               out.stride(2), ws.data_ptr(), b, hq, hkv, total, d, d ** -0.5, H.stream())
        return out
    o, _ = _ops.attention_fwd(q.transpose(1, 2), cache_k[:, :, :total], cache_v[:, :, :total], d ** -0.5)
    return o.transpose(1, 2)


def linear(x, weight, *, gemv=True, accurate=False, sliced=False, prefill_tiling=False, reference_accumulation=False):
    """``inference/kernels.py:129``: Y = X W^T; M <= 8 rows stream the weights through the GEMV
    kernel, larger M use the matrix-core GEMM.  The SM86 accumulation-order switches are accepted
    and select nothing."""
    shape = x.shape
    k = shape[-1]
    m = x.numel() // k
    n = weight.shape[0]
    if gemv and m <= 8 and x.dtype in (torch.bfloat16, torch.float16) and x.is_contiguous() and \
            weight.is_contiguous() and k % 8 == 0:
        y = torch.empty((*shape[:-1], n), device=x.device, dtype=x.dtype)
        H.call("q3_gemv", H.code(x.dtype), x.data_ptr(), k, weight.data_ptr(), y.data_ptr(), n, m, n, k, H.stream())
        return y
    return matmul(x.reshape(m, k), weight.t(), optimized=True).view(*shape[:-1], n)


_EOS_CACHE = {}


def select(logits, ids, next_token, done, position, eos, pad):
    """``inference/kernels.py:168``: greedy token (lowest index on ties), pad for finished rows,
    EOS bookkeeping; writes ids[:, position], next_token and done."""
    b, n = logits.shape
    key = (tuple(eos), logits.device)
    if key not in _EOS_CACHE:
        _EOS_CACHE[key] = torch.tensor(list(eos) or [0], dtype=torch.int64, device=logits.device)
    eos_t = _EOS_CACHE[key]
    ws = H.workspace(H.query("q3_greedy_select_workspace_bytes", b), logits.device)
    H.call("q3_greedy_select", H.code(logits.dtype), logits.data_ptr(), logits.stride(0), b, n, ws.data_ptr(),
           0 if ids is None else ids.data_ptr(), 0 if ids is None else ids.stride(0), position,
           next_token.data_ptr(), done.data_ptr(), eos_t.data_ptr(), len(eos), pad, H.stream())


def rms_norm(x, weight, eps, *, reference_accumulation=False):
    """``inference/kernels.py:176``: forward-only RMSNorm for any row count."""
    return _ops.rmsnorm_fwd(x, weight, eps)


def norm_rope(x, weight, cos, sin, eps):
    """``inference/kernels.py:188``: forward-only fused per-head RMSNorm + RoPE."""
    return _ops.norm_rope_fwd(x, weight, cos, sin, eps)
