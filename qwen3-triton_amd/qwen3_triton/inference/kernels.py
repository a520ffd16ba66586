"""Inference-only launchers: positions, KV-cache append, cached attention, small-M linear, greedy
select, and forward-only norms.  Mirrors ``qwen3_triton/inference/kernels.py`` (names and call
shapes); every op is a HIP kernel behind libq3hip.so.
"""
import ctypes

import torch

from .. import _hip as H
from ..kernels import _ops
from ..kernels.linear import matmul


def positions(batch, sequence, start, device, start_dev=None):
    """``inference/kernels.py:18``: [B,S] int64 positions start..start+S-1 (offset by the device
    int64 ``start_dev`` when given)."""
    return _ops.positions(batch, sequence, start if start_dev is None else 0, device, start_dev)


def append(k, v, cache_k, cache_v, start, start_dev=None):
    """``inference/kernels.py:33``: write k/v [B,S,Hkv,D] into the caches [B,Hkv,C,D] at ``start``
    (or at the device int64 ``start_dev``, read when the kernel runs)."""
    b, s, h, d = k.shape
    H.call("q3_kv_append", H.code(k.dtype), k.data_ptr(), v.data_ptr(), cache_k.data_ptr(), cache_v.data_ptr(), b, s,
           h, d, cache_k.shape[2], start, 0 if start_dev is None else start_dev.data_ptr(), H.stream())


def attention(q, cache_k, cache_v, start, *, split_decode=False, start_dev=None):
    """``inference/kernels.py:95``: q [B,S,Hq,D] against cache positions [0, start+S).

    S == 1 runs the split-KV decode kernel (with ``start_dev`` the length is read on the device and
    the launch spans the whole capacity, so a captured step replays at any position); S > 1
    (prefill, chunked prefill) runs the flash kernel on the cache in place (the query block is the
    suffix of the key range)."""
    b, s, hq, d = q.shape
    hkv, cap = cache_k.shape[1], cache_k.shape[2]
    total = start + s
    if s == 1 and d == 128 and q.dtype in (torch.bfloat16, torch.float16):
        out = torch.empty_like(q)
        span = cap if start_dev is not None else total
        ws = H.workspace(H.query("q3_decode_attention_workspace_bytes", b, hq, hkv, span), q.device)
        H.call("q3_decode_attention", H.code(q.dtype), q.data_ptr(), q.stride(0), q.stride(2), cache_k.data_ptr(),
               cache_v.data_ptr(), cache_k.stride(0), cache_k.stride(1), out.data_ptr(), out.stride(0),
               out.stride(2), ws.data_ptr(), b, hq, hkv, total, 0 if start_dev is None else start_dev.data_ptr(),
               cap, d, d ** -0.5, H.stream())
        return out
    if start_dev is not None:
        raise ValueError('device-resident positions are for single-token decode steps')
    o, _ = _ops.attention_fwd(q.transpose(1, 2), cache_k[:, :, :total], cache_v[:, :, :total], d ** -0.5)
    return o.transpose(1, 2)


def decode_step_attention(q, k, v, q_norm_w, k_norm_w, eps, cos, sin, cache_k, cache_v, start, start_dev=None):
    """One decode step's attention from the raw projections q [B,1,Hq,D], k, v [B,1,Hkv,D]: QK-norm,
    RoPE (cos/sin [B,1,D] at the token's position), cache append and split-KV attention in one
    kernel pair (``inference/model.py:122-125``).  Returns [B,1,Hq,D]."""
    b, s, hq, d = q.shape
    hkv, cap = cache_k.shape[1], cache_k.shape[2]
    if s != 1 or d != 128:
        raise ValueError("decode_step_attention takes one token with head_dim 128")
    out = torch.empty_like(q)
    total = start + 1
    span = cap if start_dev is not None else total
    ws = H.workspace(H.query("q3_decode_attention_workspace_bytes", b, hq, hkv, span), q.device)
    H.call("q3_decode_step_attention", H.code(q.dtype), q.data_ptr(), q.stride(0), q.stride(2), k.data_ptr(),
           v.data_ptr(), k.stride(0), k.stride(2), q_norm_w.data_ptr(), k_norm_w.data_ptr(), float(eps),
           cos.data_ptr(), sin.data_ptr(), cos.stride(0), cache_k.data_ptr(), cache_v.data_ptr(), cache_k.stride(0),
           cache_k.stride(1), out.data_ptr(), out.stride(0), out.stride(2), ws.data_ptr(), b, hq, hkv, total,
           0 if start_dev is None else start_dev.data_ptr(), cap, d, d ** -0.5, H.stream())
    return out


def linear(x, weight, *, gemv=True, accurate=False, sliced=False, prefill_tiling=False, reference_accumulation=False):
    """``inference/kernels.py:129``: Y = X W^T; M <= 8 rows stream the weights through the GEMV
    kernel, larger M use the matrix-core GEMM.  The SM86 accumulation-order switches are accepted
    and select nothing."""
    shape = x.shape
    k = shape[-1]
    m = x.numel() // k
    n = weight.shape[0]
    if gemv and m <= DECODE_MAX_ROWS and x.dtype in (torch.bfloat16, torch.float16) and x.is_contiguous() and \
            weight.is_contiguous() and k % 8 == 0:
        y = torch.empty((*shape[:-1], n), device=x.device, dtype=x.dtype)
        H.call("q3_gemv", H.code(x.dtype), x.data_ptr(), k, weight.data_ptr(), y.data_ptr(), n, m, n, k, H.stream())
        return y
    return matmul(x.reshape(m, k), weight.t(), optimized=True).view(*shape[:-1], n)


DECODE_MAX_ROWS = 16


def decode_linear_ok(x, *weights):
    """Whether the fused decode projection serves these operands (<= 16 token rows, 16-bit,
    16-byte aligned rows)."""
    k = x.shape[-1]
    return x.numel() // k <= DECODE_MAX_ROWS and x.dtype in (torch.bfloat16, torch.float16) and \
        x.is_contiguous() and k % 8 == 0 and all(w.is_contiguous() and w.dtype == x.dtype for w in weights)


def decode_linear(x, weights, *, norm_weight=None, eps=1e-6, mode=0, res=None):
    """Decode-step projection of the <= 16 token rows of ``x`` [..., K] on the matrix cores, one
    launch for: an optional RMSNorm of ``x`` (``norm_weight``), up to 3 weights sharing that input
    (mode 0, returns a list), ``res + x W^T`` (mode 1) or ``silu(x Wg^T) * (x Wu^T)`` (mode 2,
    ``weights = [Wg, Wu]``).  Replaces the reference's rms_norm + linear(s) + residual_add / swiglu
    sequence of ``inference/model.py:117-137``."""
    shape = x.shape
    k = shape[-1]
    m = x.numel() // k
    outs = [torch.empty((*shape[:-1], w.shape[0]), device=x.device, dtype=x.dtype) for w in weights]
    if mode == 2:
        outs = outs[:1]
    nseg = len(weights)
    arr_p = ctypes.c_void_p * nseg
    arr_i = ctypes.c_int64 * nseg
    ws = arr_p(*[w.data_ptr() for w in weights])
    ys = arr_p(*([o.data_ptr() for o in outs] + [outs[0].data_ptr()] * (nseg - len(outs))))
    ldy = arr_i(*[w.shape[0] for w in weights])
    ns = arr_i(*[w.shape[0] for w in weights])
    H.call("q3_decode_linear", H.code(x.dtype), x.data_ptr(), k, m, k,
           0 if norm_weight is None else norm_weight.data_ptr(), float(eps), mode, nseg, ws, ys, ldy, ns,
           0 if res is None else res.data_ptr(), 0 if res is None else res.shape[-1], H.stream())
    return outs if mode == 0 else outs[0]


_EOS_CACHE = {}


def select(logits, ids, next_token, done, position, eos, pad, position_dev=None):
    """``inference/kernels.py:168``: greedy token (lowest index on ties), pad for finished rows,
    EOS bookkeeping; writes ids[:, position (+ *position_dev)], next_token and done."""
    b, n = logits.shape
    key = (tuple(eos), logits.device)
    if key not in _EOS_CACHE:
        _EOS_CACHE[key] = torch.tensor(list(eos) or [0], dtype=torch.int64, device=logits.device)
    eos_t = _EOS_CACHE[key]
    ws = H.workspace(H.query("q3_greedy_select_workspace_bytes", b), logits.device)
    H.call("q3_greedy_select", H.code(logits.dtype), logits.data_ptr(), logits.stride(0), b, n, ws.data_ptr(),
           0 if ids is None else ids.data_ptr(), 0 if ids is None else ids.stride(0), position,
           0 if position_dev is None else position_dev.data_ptr(), next_token.data_ptr(), done.data_ptr(),
           eos_t.data_ptr(), len(eos), pad, H.stream())


def advance(counter, by):
    """counter (device int64) += by, as a kernel on the current stream."""
    H.call("q3_advance", counter.data_ptr(), by, H.stream())


def rms_norm(x, weight, eps, *, reference_accumulation=False):
    """``inference/kernels.py:176``: forward-only RMSNorm for any row count."""
    return _ops.rmsnorm_fwd(x, weight, eps)


def norm_rope(x, weight, cos, sin, eps):
    """``inference/kernels.py:188``: forward-only fused per-head RMSNorm + RoPE."""
    return _ops.norm_rope_fwd(x, weight, cos, sin, eps)


def sliced_linear(x, weight):
    """``inference/kernels.py:213``: Y = x W^T for ONE token row (decode GEMV).  The reference's
    two-accumulator SM86 slicing is an accumulation-order choice; here it is the streaming decode
    kernel."""
    if x.numel() != x.shape[-1] or not x.is_contiguous() or not weight.is_contiguous():
        raise ValueError('one contiguous token row and a row-major weight are required')
    if x.dtype != torch.bfloat16 or weight.dtype != x.dtype or x.device != weight.device or not x.is_cuda or \
            x.shape[-1] != weight.shape[1]:
        raise ValueError('matching bf16 ROCm input and [N, K] weight required')
    return linear(x, weight, gemv=True)


def tiled_prefill_gate_up(x, gate_weight, up_weight):
    """``inference/kernels.py:222``: silu(x Wg^T) * (x Wu^T) for a short prefill chunk, forward only
    (the dual-weight GEMM of ``mlp_precision``; any row count, not only the reference's M = 65)."""
    n, k = gate_weight.shape
    if x.shape[-1] != k or up_weight.shape != gate_weight.shape:
        raise ValueError('x [..., K] with matching [N, K] gate/up weights required')
    if x.dtype != torch.bfloat16 or not x.is_cuda or \
            any(t.device != x.device or t.dtype != x.dtype or not t.is_contiguous() for t in (x, gate_weight, up_weight)):
        raise ValueError('matching contiguous bf16 ROCm inputs required')
    from ..kernels.mlp_precision import gate_up_swiglu
    with torch.no_grad():
        return gate_up_swiglu(x, gate_weight, up_weight, optimized=True)
