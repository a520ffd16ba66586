"""Functional (non-autograd) launchers over libq3hip.so.

Each function validates shapes on the host, allocates its outputs with the torch caching
allocator on the input's device, and launches on the current stream.  The autograd modules of
this package (named after the reference's ``qwen3_triton/kernels/*`` and ``ops/triton/*``)
are built on these.
"""
from __future__ import annotations

import torch

from .. import _hip as H


def _cont(t: torch.Tensor, what: str) -> torch.Tensor:
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous; no hidden layout copy")
    return t


# ---------------------------------------------------------------- norms
def rmsnorm_fwd(x, w, eps):
    h = w.numel()
    y = torch.empty_like(x)
    H.call("q3_rmsnorm_fwd", H.code(x.dtype), x.data_ptr(), w.data_ptr(), y.data_ptr(), x.numel() // h, h,
           float(eps), H.stream())
    return y


def rmsnorm_bwd(x, w, dy, eps):
    h = w.numel()
    rows = x.numel() // h
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    ws = H.workspace(H.query("q3_rmsnorm_bwd_workspace_bytes", rows, h), x.device)
    H.call("q3_rmsnorm_bwd", H.code(x.dtype), x.data_ptr(), w.data_ptr(), dy.data_ptr(), dx.data_ptr(),
           dw.data_ptr(), ws.data_ptr(), rows, h, float(eps), H.stream())
    return dx, dw


def norm_rope_fwd(x, w, cos, sin, eps):
    """x [B,S,heads,D] (or [tokens,heads,D]); cos/sin [B,S,D]."""
    d, heads = x.shape[-1], x.shape[-2]
    tokens = x.numel() // (d * heads)
    y = torch.empty_like(x)
    H.call("q3_norm_rope_fwd", H.code(x.dtype), x.data_ptr(), w.data_ptr(), cos.data_ptr(), sin.data_ptr(),
           y.data_ptr(), tokens, heads, d, float(eps), H.stream())
    return y


def norm_rope_bwd(x, w, cos, sin, dy, eps):
    d, heads = x.shape[-1], x.shape[-2]
    tokens = x.numel() // (d * heads)
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    ws = H.workspace(H.query("q3_norm_rope_bwd_workspace_bytes", tokens, heads, d), x.device)
    H.call("q3_norm_rope_bwd", H.code(x.dtype), x.data_ptr(), w.data_ptr(), cos.data_ptr(), sin.data_ptr(),
           dy.data_ptr(), dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), tokens, heads, d, float(eps), H.stream())
    return dx, dw


# ---------------------------------------------------------------- rope
def rope_tables(position_ids, inv_freq, dtype):
    d = inv_freq.numel() * 2
    cos = torch.empty((*position_ids.shape, d), device=position_ids.device, dtype=dtype)
    sin = torch.empty_like(cos)
    H.call("q3_rope_tables", H.code(dtype), position_ids.data_ptr(), int(position_ids.dtype == torch.int64),
           inv_freq.data_ptr(), cos.data_ptr(), sin.data_ptr(), position_ids.numel(), d, H.stream())
    return cos, sin


def rope_apply(x, cos, sin, *, layout, backward):
    """layout 0: x [B,S,H,D]; layout 1: x [B,H,S,D]; cos/sin [B,S,D]."""
    b, d = x.shape[0], x.shape[3]
    seq, heads = (x.shape[1], x.shape[2]) if layout == 0 else (x.shape[2], x.shape[1])
    y = torch.empty_like(x)
    H.call("q3_rope_apply", H.code(x.dtype), x.data_ptr(), cos.data_ptr(), sin.data_ptr(), y.data_ptr(), b, seq,
           heads, d, layout, int(backward), H.stream())
    return y


# ---------------------------------------------------------------- swiglu / elementwise
def swiglu_fwd(g, u):
    y = torch.empty_like(g)
    H.call("q3_swiglu_fwd", H.code(g.dtype), g.data_ptr(), u.data_ptr(), y.data_ptr(), g.numel(), H.stream())
    return y


def swiglu_bwd(g, u, dy):
    dg, du = torch.empty_like(g), torch.empty_like(u)
    H.call("q3_swiglu_bwd", H.code(g.dtype), g.data_ptr(), u.data_ptr(), dy.data_ptr(), dg.data_ptr(),
           du.data_ptr(), g.numel(), H.stream())
    return dg, du


def add(a, b, out=None):
    c = torch.empty_like(a) if out is None else out
    H.call("q3_add", H.code(a.dtype), a.data_ptr(), b.data_ptr(), c.data_ptr(), a.numel(), H.stream())
    return c


def cast(x, dtype):
    y = torch.empty(x.shape, device=x.device, dtype=dtype)
    if x.numel():
        H.call("q3_cast", H.code(x.dtype), H.code(dtype), x.data_ptr(), y.data_ptr(), x.numel(), H.stream())
    return y


def fill_(x, value):
    if x.numel():
        H.call("q3_fill", H.code(x.dtype), x.data_ptr(), float(value), x.numel(), H.stream())
    return x


def positions(batch, seq, start, device):
    out = torch.empty((batch, seq), device=device, dtype=torch.int64)
    H.call("q3_positions", out.data_ptr(), batch, seq, start, H.stream())
    return out


def transpose_last2(x):
    """[..., R, C] -> contiguous [..., C, R] (a layout change done by a HIP kernel)."""
    r, c = x.shape[-2], x.shape[-1]
    batch = x.numel() // (r * c) if x.numel() else 0
    y = torch.empty((*x.shape[:-2], c, r), device=x.device, dtype=x.dtype)
    if batch:
        H.call("q3_transpose", H.code(x.dtype), x.data_ptr(), y.data_ptr(), batch, r, c, H.stream())
    return y


# ---------------------------------------------------------------- embedding
def embedding_fwd(ids, w, bad=None):
    v, h = w.shape
    y = torch.empty((*ids.shape, h), device=w.device, dtype=w.dtype)
    H.call("q3_embedding_fwd", H.code(w.dtype), ids.data_ptr(), int(ids.dtype == torch.int64), w.data_ptr(),
           y.data_ptr(), 0 if bad is None else bad.data_ptr(), ids.numel(), v, h, H.stream())
    return y


def embedding_bwd(ids, dy, vocab, dtype):
    h = dy.shape[-1]
    dw = torch.empty((vocab, h), device=dy.device, dtype=dtype)
    ws = H.workspace(H.query("q3_embedding_bwd_workspace_bytes", ids.numel()), dy.device)
    H.call("q3_embedding_bwd", H.code(dtype), ids.data_ptr(), int(ids.dtype == torch.int64), dy.data_ptr(),
           dw.data_ptr(), ws.data_ptr(), ids.numel(), vocab, h, H.stream())
    return dw
