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


def rmsnorm_bwd_add(x, w, dy, dres, eps):
    """dx = dres + the RMSNorm input gradient (one kernel), dw."""
    h = w.numel()
    rows = x.numel() // h
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    ws = H.workspace(H.query("q3_rmsnorm_bwd_workspace_bytes", rows, h), x.device)
    H.call("q3_rmsnorm_bwd_add", H.code(x.dtype), x.data_ptr(), w.data_ptr(), dy.data_ptr(), dres.data_ptr(),
           dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), rows, h, float(eps), H.stream())
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


def norm_rope_qk_ok(q, k, d):
    """Whether q3_norm_rope_qk_fwd / _bwd take this shape (the vector path of both tensors)."""
    v = 4 if q.dtype == torch.float32 else 8
    return d % 2 == 0 and (d // 2) % v == 0 and d // v in (8, 16, 32)


def norm_rope_qk_fwd(q, k, wq, wk, cos, sin, eps):
    """q [.., hq, d], k [.., hk, d] over the same tokens; one launch for both."""
    d, hq, hk = q.shape[-1], q.shape[-2], k.shape[-2]
    tokens = q.numel() // (d * hq)
    yq, yk = torch.empty_like(q), torch.empty_like(k)
    H.call("q3_norm_rope_qk_fwd", H.code(q.dtype), q.data_ptr(), k.data_ptr(), wq.data_ptr(), wk.data_ptr(),
           cos.data_ptr(), sin.data_ptr(), yq.data_ptr(), yk.data_ptr(), tokens, hq, hk, d, float(eps), H.stream())
    return yq, yk


def norm_rope_qk_cache_fwd(q, k, v, wq, wk, cos, sin, cache_k, cache_v, start, eps):
    """Prefill chunk: q / k / v [B, S, h, d] contiguous; returns the normed + rotated q and writes the
    normed + rotated k and the raw v into the [B, hk, capacity, d] caches at ``start``."""
    b, s, hq, d = q.shape
    hk = k.shape[2]
    yq = torch.empty_like(q)
    H.call("q3_norm_rope_qk_cache_fwd", H.code(q.dtype), q.data_ptr(), k.data_ptr(), v.data_ptr(), wq.data_ptr(),
           wk.data_ptr(), cos.data_ptr(), sin.data_ptr(), yq.data_ptr(), cache_k.data_ptr(), cache_v.data_ptr(), b, s,
           hq, hk, d, cache_k.shape[2], start, float(eps), H.stream())
    return yq


def norm_rope_qk_bwd(q, k, wq, wk, cos, sin, dyq, dyk, eps):
    d, hq, hk = q.shape[-1], q.shape[-2], k.shape[-2]
    tokens = q.numel() // (d * hq)
    dxq, dxk = torch.empty_like(q), torch.empty_like(k)
    dw = torch.empty((2, d), device=q.device, dtype=wq.dtype)
    ws = H.workspace(H.query("q3_norm_rope_qk_bwd_workspace_bytes", tokens, hq, hk, d), q.device)
    H.call("q3_norm_rope_qk_bwd", H.code(q.dtype), q.data_ptr(), k.data_ptr(), wq.data_ptr(), wk.data_ptr(),
           cos.data_ptr(), sin.data_ptr(), dyq.data_ptr(), dyk.data_ptr(), dxq.data_ptr(), dxk.data_ptr(),
           dw.data_ptr(), ws.data_ptr(), tokens, hq, hk, d, float(eps), H.stream())
    return dxq, dxk, dw[0], dw[1]


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


def _rows_strided(t):
    return t.ndim == 2 and t.stride(1) == 1


def swiglu_bwd_into(g, u, dy, dg, du):
    """SwiGLU backward on [rows, cols] operands whose rows may sit at their own strides (dg and du can
    be the two halves of one [rows, 2*cols] buffer)."""
    for t in (g, u, dy, dg, du):
        if not _rows_strided(t) or t.shape != g.shape:
            raise ValueError("matching [rows, cols] row-strided operands required")
    r, c = g.shape
    H.call("q3_swiglu_bwd_2d", H.code(g.dtype), g.data_ptr(), g.stride(0), u.data_ptr(), u.stride(0), dy.data_ptr(),
           dy.stride(0), dg.data_ptr(), dg.stride(0), du.data_ptr(), du.stride(0), r, c, H.stream())
    return dg, du


def copy_into(src, dst):
    """dst[:, :] = src for [rows, cols] blocks at their own row strides."""
    if not (_rows_strided(src) and _rows_strided(dst)) or src.shape != dst.shape or src.dtype != dst.dtype:
        raise ValueError("matching [rows, cols] row-strided operands required")
    H.call("q3_copy2d", H.code(src.dtype), src.data_ptr(), src.stride(0), dst.data_ptr(), dst.stride(0),
           src.shape[0], src.shape[1], H.stream())
    return dst


def transpose_into(src, dst):
    """dst = src^T for src [R, C] and dst [C, R] at their own row strides; dst may be a column block of
    a wider matrix (nothing outside it is written)."""
    r, c = src.shape
    if not (_rows_strided(src) and _rows_strided(dst)) or dst.shape != (c, r) or src.dtype != dst.dtype:
        raise ValueError("[R, C] source and [C, R] row-strided destination required")
    H.call("q3_transpose2d", H.code(src.dtype), src.data_ptr(), src.stride(0), dst.data_ptr(), dst.stride(0), r, c,
           H.stream())
    return dst


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


def positions(batch, seq, start, device, start_dev=None):
    """[B,S] int64 positions start + s (+ the device int64 ``start_dev`` when given)."""
    out = torch.empty((batch, seq), device=device, dtype=torch.int64)
    H.call("q3_positions", out.data_ptr(), batch, seq, start, 0 if start_dev is None else start_dev.data_ptr(),
           H.stream())
    return out


def transpose_last2(x, pad_to=1):
    """[..., R, C] -> contiguous [..., C, Rp] with Rp = R rounded up to ``pad_to`` (pad zero-filled);
    a layout change done by a HIP kernel."""
    r, c = x.shape[-2], x.shape[-1]
    rp = -(-r // pad_to) * pad_to
    batch = x.numel() // (r * c) if x.numel() else 0
    y = torch.empty((*x.shape[:-2], c, rp), device=x.device, dtype=x.dtype)
    if batch:
        H.call("q3_transpose", H.code(x.dtype), x.data_ptr(), y.data_ptr(), batch, r, c, rp, H.stream())
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


# ---------------------------------------------------------------- attention
def attention_mfma(dtype, d):
    return bool(H.query("q3_attention_mfma_supported", H.code(dtype), d))


def _bhsd_strides(t):
    if t.stride(3) != 1:
        raise ValueError("attention operands need a contiguous head dimension")
    return t.stride(0), t.stride(1), t.stride(2)


def seq_major(x, pad_to=16):
    """[B,H,L,D]-indexed view (any b/h/s strides) -> contiguous [B,H,D,Lp], Lp = L rounded up to
    ``pad_to``, zero pad (the sequence-contiguous operand copy of the matrix-core attention)."""
    b, h, l, d = x.shape
    lp = -(-l // pad_to) * pad_to
    y = torch.empty((b, h, d, lp), device=x.device, dtype=x.dtype)
    H.call("q3_attention_seq_major", H.code(x.dtype), x.data_ptr(), *_bhsd_strides(x), y.data_ptr(), lp, b, h, l, d,
           H.stream())
    return y


def attention_fwd(q, k, v, scale):
    """Causal GQA attention on [B,H,L,D]-indexed views (D contiguous; batch/head/position strides free,
    k and v sharing theirs) -> (o laid out like q, lse [B,Hq,Lq] fp32)."""
    b, hq, lq, d = q.shape
    hkv, lk = k.shape[1], k.shape[2]
    if v.stride() != k.stride():
        raise ValueError("k and v must share strides")
    o = torch.empty_like(q)
    if o.stride() != q.stride():
        o = torch.empty_strided(q.shape, q.stride(), device=q.device, dtype=q.dtype)
    lse = torch.empty((b, hq, lq), device=q.device, dtype=torch.float32)
    vt, ldvt = None, 0
    if attention_mfma(q.dtype, d):
        vt = seq_major(v)
        ldvt = vt.shape[-1]
    H.call("q3_attention_fwd", H.code(q.dtype), q.data_ptr(), *_bhsd_strides(q), k.data_ptr(), v.data_ptr(),
           *_bhsd_strides(k), 0 if vt is None else vt.data_ptr(), ldvt, o.data_ptr(), lse.data_ptr(), b, hq, hkv,
           lq, lk, d, float(scale), H.stream())
    return o, lse


def _like(t, ref):
    """t re-laid out with ref's strides (a copy only when they differ)."""
    if t.stride() == ref.stride():
        return t
    out = torch.empty_strided(ref.shape, ref.stride(), device=ref.device, dtype=ref.dtype)
    out.copy_(t)
    return out


def attention_bwd(q, k, v, o, lse, do, scale):
    b, hq, lq, d = q.shape
    hkv, lk = k.shape[1], k.shape[2]
    o, do = _like(o, q), _like(do, q)
    v = _like(v, k)
    dq = torch.empty_strided(q.shape, q.stride(), device=q.device, dtype=q.dtype)
    dk = torch.empty_strided(k.shape, k.stride(), device=k.device, dtype=k.dtype)
    dv = torch.empty_strided(k.shape, k.stride(), device=k.device, dtype=k.dtype)
    delta = torch.empty((b, hq, lq), device=q.device, dtype=torch.float32)
    qt = kt = dot = None
    ldq = ldk = 0
    if attention_mfma(q.dtype, d):
        kt = seq_major(k)
        ldk = kt.shape[-1]
        if d != 128:  # head_dim 128 reads Q and dO transposed in LDS
            qt, dot = seq_major(q), seq_major(do)
            ldq = qt.shape[-1]
    p = (lambda t: 0 if t is None else t.data_ptr())
    H.call("q3_attention_bwd", H.code(q.dtype), q.data_ptr(), *_bhsd_strides(q), k.data_ptr(), v.data_ptr(),
           *_bhsd_strides(k), o.data_ptr(), do.data_ptr(), lse.data_ptr(), p(qt), ldq, p(kt), ldk, p(dot),
           delta.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), b, hq, hkv, lq, lk, d, float(scale),
           H.stream())
    return dq, dk, dv


# ---------------------------------------------------------------- cross-entropy
def ce_shift_labels(labels, ignore_index):
    b, s = labels.shape
    tgt = torch.empty(b * s, device=labels.device, dtype=torch.int64)
    H.call("q3_ce_shift_labels", labels.data_ptr(), tgt.data_ptr(), b, s, int(ignore_index), H.stream())
    return tgt


class CEState:
    """Per-row partial statistics of a chunked causal CE (chunk-major [nchunks][rows])."""

    def __init__(self, rows, nchunks, device):
        f = dict(device=device, dtype=torch.float32)
        self.rows, self.nchunks = rows, nchunks
        self.m = torch.empty((nchunks, rows), **f)
        self.s = torch.empty((nchunks, rows), **f)
        self.pick = torch.empty(rows, **f)
        self.lse = torch.empty(rows, **f)
        self.loss_rows = torch.empty(rows, **f)
        self.loss = torch.empty((), **f)
        self.count = torch.empty((), **f)

    def stats(self, chunk, z, ld, n, col0, tgt):
        H.call("q3_ce_chunk_stats", H.code(z.dtype), z.data_ptr(), ld, n, col0, tgt.data_ptr(),
               self.m[chunk].data_ptr(), self.s[chunk].data_ptr(), self.pick.data_ptr(), self.rows, H.stream())

    def gemm_stats(self, part0, x, w, col0, n, tgt):
        """Logits x . w[col0:col0+n]^T and their statistics in one matrix-core kernel: partials
        part0 .. part0 + ceil(n / 128) - 1 (128 logit columns each) and the target logits."""
        t, h = x.shape
        H.call("q3_gemm_nt_ce_stats", H.code(x.dtype), x.data_ptr(), x.stride(0), w[col0:].data_ptr(), w.stride(0),
               t, n, h, col0, tgt.data_ptr(), self.m.data_ptr(), self.s.data_ptr(), self.pick.data_ptr(), part0,
               self.rows, H.stream())

    def gemm_stats_store(self, part0, x, w, col0, n, tgt, z):
        """gemm_stats that also stores the logits in x's dtype into z[:, :n] (statistics from the stored,
        rounded values)."""
        t, h = x.shape
        H.call("q3_gemm_nt_ce_stats_store", H.code(x.dtype), x.data_ptr(), x.stride(0), w[col0:].data_ptr(),
               w.stride(0), t, n, h, col0, tgt.data_ptr(), self.m.data_ptr(), self.s.data_ptr(),
               self.pick.data_ptr(), part0, self.rows, z.data_ptr(), z.stride(0), H.stream())

    def finish(self, tgt, vocab, ignore_index, check=True):
        capturing = torch.cuda.is_current_stream_capturing()
        bad = None if (capturing or not check) else torch.zeros((), device=tgt.device, dtype=torch.int32)
        H.call("q3_ce_finish", self.m.data_ptr(), self.s.data_ptr(), self.nchunks, self.pick.data_ptr(),
               tgt.data_ptr(), self.lse.data_ptr(), self.loss_rows.data_ptr(), 0 if bad is None else bad.data_ptr(),
               self.loss.data_ptr(), self.count.data_ptr(), self.rows, vocab, int(ignore_index), H.stream())
        if bad is not None and bool(bad.item()):
            raise ValueError('CE label out of range')
        return self.loss


def gemm_ce_grad(x, w, col0, n, tgt, lse, count, up, dz, vocab, ignore_index, dzt=None):
    """dz[:, :n] = CE gradient of the logits x . w[col0:col0+n]^T (matrix cores; fp32 logits stay in
    registers), and dzt[:n, :] = its transpose when given.  x [T, H] and w [V, H] K-contiguous
    bf16/fp16, H % 64 == 0."""
    t, h = x.shape
    H.call("q3_gemm_nt_ce_grad", H.code(x.dtype), x.data_ptr(), x.stride(0), w[col0:].data_ptr(), w.stride(0),
           dz.data_ptr(), dz.stride(0), 0 if dzt is None else dzt.data_ptr(), 0 if dzt is None else dzt.stride(0),
           t, n, h, col0, tgt.data_ptr(), lse.data_ptr(), count.data_ptr(),
           0 if up is None else up.data_ptr(), vocab, int(ignore_index), H.stream())


def ce_grad_transposed_ok(x, t, n, lddz, dz, dzt):
    """Whether q3_gemm_nt_ce_grad can write the transposed dz copy for this chunk."""
    return t % 256 == 0 and n % 256 == 0 and (t // 256) * (n // 256) >= 256 and lddz % 8 == 0 and \
        dz.data_ptr() % 16 == 0 and dzt.stride(0) % 8 == 0 and dzt.data_ptr() % 16 == 0


def ce_grad_t(z, n, col0, tgt, lse, count, up, dz, dzt, vocab, ignore_index):
    """dz[:, :n] (may be z itself) and dzt[:n, :] from stored 16-bit logits z[:, :n]."""
    H.call("q3_ce_chunk_grad_t", H.code(z.dtype), z.data_ptr(), z.stride(0), n, col0, tgt.data_ptr(), lse.data_ptr(),
           count.data_ptr(), 0 if up is None else up.data_ptr(), dz.data_ptr(), dz.stride(0), dzt.data_ptr(),
           dzt.stride(0), tgt.numel(), vocab, int(ignore_index), H.stream())


def ce_grad(z, ld, n, col0, tgt, lse, count, up, dz, ldo, vocab, ignore_index):
    rows = tgt.numel()
    H.call("q3_ce_chunk_grad", H.code(z.dtype), H.code(dz.dtype), z.data_ptr(), ld, n, col0, tgt.data_ptr(),
           lse.data_ptr(), count.data_ptr(), 0 if up is None else up.data_ptr(), dz.data_ptr(), ldo, rows, vocab,
           int(ignore_index), H.stream())
