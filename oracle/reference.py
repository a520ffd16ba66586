"""fp32/fp64 PyTorch-CPU restatement of the reference math (TEST INFRASTRUCTURE).

All functions compute in ``dtype`` (default float32; tests use float64 to pin
rounding-free values) and never call anything outside ``torch``.  Citations are
to files of wuyii8941/qwen3-triton.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

__all__ = [
    "rms_norm_reference", "rms_norm_backward_reference",
    "rotate_half_reference", "inverse_rotate_half_reference",
    "apply_rope_reference", "apply_rope_backward_reference",
    "rope_inv_freq", "rotary_tables_reference",
    "fused_qk_norm_rope_reference", "fused_qk_norm_rope_backward_reference",
    "swiglu_reference", "swiglu_backward_reference",
    "scaled_dot_product_attention_reference", "attention_lse_reference",
    "scaled_dot_product_attention_backward_reference",
    "causal_cross_entropy_reference", "causal_cross_entropy_backward_reference",
    "lm_head_cross_entropy_reference",
    "embedding_backward_reference",
    "OracleConfig", "init_params", "decoder_layer_reference", "model_forward_reference",
    "greedy_generate_reference", "argmax_lowest_reference", "cached_decode_reference",
]


# --------------------------------------------------------------------------- norms
def rms_norm_reference(x, weight, eps, *, dtype=torch.float32):
    """``ops/reference/rms_norm.py:6-13``: y = x*rsqrt(mean(x^2)+eps)*w over the last dim."""
    xf = x.to(dtype)
    inv = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return xf * inv * weight.to(dtype)


def rms_norm_backward_reference(x, weight, grad_y, eps, *, dtype=torch.float32):
    """Explicit RMSNorm backward, ``ops/reference/fused_qk_norm_rope.py:63-76``.

    dx = (g*w - x*inv^2*mean(g*w*x))*inv ; dw = sum_rows g*x*inv.
    """
    xf, wf, gf = x.to(dtype), weight.to(dtype), grad_y.to(dtype)
    inv = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    weighted = gf * wf
    correction = (weighted * xf).mean(dim=-1, keepdim=True)
    dx = (weighted - xf * inv.square() * correction) * inv
    dw = (gf * xf * inv).reshape(-1, x.shape[-1]).sum(dim=0)
    return dx, dw


# --------------------------------------------------------------------------- rope
def rotate_half_reference(x):
    """``ops/reference/rope.py:6-9``: cat(-second_half, first_half)."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def inverse_rotate_half_reference(x):
    """``ops/reference/rope.py:30-33``: the transpose of rotate_half, cat(second, -first)."""
    h = x.shape[-1] // 2
    return torch.cat((x[..., h:], -x[..., :h]), dim=-1)


def apply_rope_reference(q, k, cos, sin, *, dtype=torch.float32):
    """``ops/reference/rope.py:12-27``; q/k [B,H,S,D], cos/sin [B,S,D]."""
    c, s = cos.to(dtype).unsqueeze(1), sin.to(dtype).unsqueeze(1)
    q, k = q.to(dtype), k.to(dtype)
    return q * c + rotate_half_reference(q) * s, k * c + rotate_half_reference(k) * s


def apply_rope_backward_reference(gq, gk, cos, sin, *, dtype=torch.float32):
    """``ops/reference/rope.py:36-55``: dx = g*cos + rotate_half^T(g*sin)."""
    c, s = cos.to(dtype).unsqueeze(1), sin.to(dtype).unsqueeze(1)
    gq, gk = gq.to(dtype), gk.to(dtype)
    return (gq * c + inverse_rotate_half_reference(gq * s),
            gk * c + inverse_rotate_half_reference(gk * s))


def rope_inv_freq(theta, head_dim):
    """``qwen3_triton/_model.py:54`` / ``model/qwen_tiny.py:48``: 1/theta^(2i/D) in fp32."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))


def rotary_tables_reference(position_ids, inv_freq, *, dtype=torch.float32):
    """``model/qwen_tiny.py:53-63`` and ``qwen3_triton/kernels/rotary.py:12-17``.

    angle = fp32(pos) * fp32(inv_freq), duplicated over both halves; cos/sin of it.
    """
    ang = position_ids.to(torch.float32)[..., None] * inv_freq.to(torch.float32)
    emb = torch.cat((ang, ang), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def fused_qk_norm_rope_reference(q, k, qw, kw, cos, sin, eps=1e-6, *, dtype=torch.float32):
    """``ops/reference/fused_qk_norm_rope.py:9-32``; q/k [B,S,H,D], cos/sin [B,S,D]."""
    qn = rms_norm_reference(q, qw, eps, dtype=dtype)
    kn = rms_norm_reference(k, kw, eps, dtype=dtype)
    qr, kr = apply_rope_reference(qn.transpose(1, 2), kn.transpose(1, 2), cos, sin, dtype=dtype)
    return qr.transpose(1, 2), kr.transpose(1, 2)


def fused_qk_norm_rope_backward_reference(q, k, qw, kw, cos, sin, gq, gk, eps=1e-6, *, dtype=torch.float32):
    """``ops/reference/fused_qk_norm_rope.py:35-80``: rope backward then RMSNorm backward."""
    gqn, gkn = apply_rope_backward_reference(gq.transpose(1, 2), gk.transpose(1, 2), cos, sin, dtype=dtype)
    dq, dqw = rms_norm_backward_reference(q, qw, gqn.transpose(1, 2), eps, dtype=dtype)
    dk, dkw = rms_norm_backward_reference(k, kw, gkn.transpose(1, 2), eps, dtype=dtype)
    return dq, dk, dqw, dkw


# --------------------------------------------------------------------------- swiglu
def swiglu_reference(gate, up, *, dtype=torch.float32):
    """``ops/reference/swiglu.py:9-21``: silu(g)*u with silu(g) = g*sigmoid(g)."""
    g, u = gate.to(dtype), up.to(dtype)
    return g * torch.sigmoid(g) * u


def swiglu_backward_reference(gate, up, dy, *, dtype=torch.float32):
    """``qwen3_triton/kernels/activation.py:14-19``: dg = dy*u*s*(1+g*(1-s)), du = dy*g*s."""
    g, u, d = gate.to(dtype), up.to(dtype), dy.to(dtype)
    s = torch.sigmoid(g)
    return d * u * s * (1 + g * (1 - s)), d * g * s


# --------------------------------------------------------------------------- attention
def _expand_kv(k, v, hq):
    hk = k.shape[1]
    if hq % hk:
        raise ValueError("q_heads must be divisible by kv_heads")
    g = hq // hk
    return k.repeat_interleave(g, dim=1), v.repeat_interleave(g, dim=1), g


def _causal_scores(q, k, scale, is_causal):
    sc = torch.matmul(q, k.transpose(-2, -1)) * scale
    if is_causal:
        ql, kl = q.shape[-2], k.shape[-2]
        qpos = torch.arange(ql) + (kl - ql)
        allowed = torch.arange(kl)[None, :] <= qpos[:, None]
        sc = sc.masked_fill(~allowed, float("-inf"))
    return sc


def scaled_dot_product_attention_reference(q, k, v, *, is_causal=True, scale=None, dtype=torch.float32):
    """``ops/reference/attention.py:10-54``: softmax(QK^T*s + causal)V with GQA head mapping.

    Causal uses the suffix-offset form (query i sees keys <= i + Lk - Lq), ``:46-51``.
    """
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    ke, ve, _ = _expand_kv(k, v, q.shape[1])
    p = torch.softmax(_causal_scores(q, ke, scale, is_causal), dim=-1)
    return torch.matmul(p, ve)


def attention_lse_reference(q, k, *, is_causal=True, scale=None, dtype=torch.float32):
    """Row logsumexp of the scaled, masked scores (``tests/test_attention_triton.py:36-47``)."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    q, k = q.to(dtype), k.to(dtype)
    ke, _, _ = _expand_kv(k, k, q.shape[1])
    return torch.logsumexp(_causal_scores(q, ke, scale, is_causal), dim=-1)


def scaled_dot_product_attention_backward_reference(q, k, v, grad_out, *, is_causal=True, scale=None,
                                                    dtype=torch.float32):
    """``ops/reference/attention.py:57-124``: explicit dV=P^T dO, dS=P*(dP-rowsum(dP*P)), dQ, dK."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    q, k, v, do = q.to(dtype), k.to(dtype), v.to(dtype), grad_out.to(dtype)
    b, hq, lq, d = q.shape
    hk, lk = k.shape[1], k.shape[2]
    ke, ve, g = _expand_kv(k, v, hq)
    p = torch.softmax(_causal_scores(q, ke, scale, is_causal), dim=-1)
    dv = torch.matmul(p.transpose(-2, -1), do)
    dp = torch.matmul(do, ve.transpose(-2, -1))
    ds = p * (dp - (dp * p).sum(dim=-1, keepdim=True))
    dq = torch.matmul(ds, ke) * scale
    dk = torch.matmul(ds.transpose(-2, -1), q) * scale
    dk = dk.view(b, hk, g, lk, d).sum(dim=2)
    dv = dv.view(b, hk, g, lk, d).sum(dim=2)
    return dq, dk, dv


# --------------------------------------------------------------------------- loss
def causal_cross_entropy_reference(logits, labels, *, ignore_index=-100, dtype=torch.float32):
    """``qwen3_triton/kernels/loss.py:7-32`` and ``model/qwen_tiny.py:224-227``.

    Row (b, s<S-1) predicts labels[b, s+1]; loss = mean over non-ignored rows of lse - z_label.
    """
    z = logits[:, :-1, :].to(dtype).reshape(-1, logits.shape[-1])
    y = labels[:, 1:].reshape(-1)
    valid = y != ignore_index
    lse = torch.logsumexp(z, dim=-1)
    picked = z.gather(1, torch.where(valid, y, 0)[:, None])[:, 0]
    per = torch.where(valid, lse - picked, torch.zeros_like(lse))
    return per.sum() / valid.sum().to(dtype)


def causal_cross_entropy_backward_reference(logits, labels, grad=1.0, *, ignore_index=-100, dtype=torch.float32):
    """``qwen3_triton/kernels/loss.py:35-44``: dz = (softmax - onehot)*grad/count; last position and
    ignored rows get zero."""
    b, s, v = logits.shape
    z = logits.to(dtype)
    out = torch.zeros((b, s, v), dtype=dtype)
    y = labels[:, 1:]
    valid = y != ignore_index
    count = valid.sum().to(dtype)
    p = torch.softmax(z[:, :-1, :], dim=-1)
    p = p - torch.nn.functional.one_hot(torch.where(valid, y, 0), v).to(dtype)
    p = p * valid[..., None].to(dtype) * (grad / count)
    out[:, :-1, :] = p
    return out


def lm_head_cross_entropy_reference(hidden, weight, labels, *, ignore_index=-100, dtype=torch.float32,
                                    chunk=16384, want_grad=False):
    """Fused LM-head + causal CE (new in this build; composes ``kernels/linear.py:80-101`` with
    ``kernels/loss.py:46-71``).  Computed per vocabulary chunk so the full logits are never held.

    Returns loss, and with ``want_grad`` also (d_hidden, d_weight) for an upstream gradient of 1.
    """
    b, s, h = hidden.shape
    x = hidden.to(dtype).reshape(b * s, h)
    y = torch.cat([labels[:, 1:], torch.full((b, 1), ignore_index, dtype=labels.dtype)], dim=1).reshape(-1)
    valid = y != ignore_index
    n = weight.shape[0]
    m = torch.full((b * s,), float("-inf"), dtype=dtype)
    l = torch.zeros((b * s,), dtype=dtype)
    picked = torch.zeros((b * s,), dtype=dtype)
    for c0 in range(0, n, chunk):
        w = weight[c0:c0 + chunk].to(dtype)
        z = x @ w.T
        cm = z.max(dim=1).values
        nm = torch.maximum(m, cm)
        l = l * torch.exp(m - nm) + torch.exp(z - nm[:, None]).sum(dim=1)
        m = nm
        inside = valid & (y >= c0) & (y < c0 + w.shape[0])
        idx = torch.where(inside, y - c0, 0)
        picked = torch.where(inside, z.gather(1, idx[:, None])[:, 0], picked)
    lse = m + torch.log(l)
    count = valid.sum().to(dtype)
    loss = torch.where(valid, lse - picked, torch.zeros_like(lse)).sum() / count
    if not want_grad:
        return loss
    dx = torch.zeros_like(x)
    dw = torch.zeros((n, h), dtype=dtype)
    for c0 in range(0, n, chunk):
        w = weight[c0:c0 + chunk].to(dtype)
        z = x @ w.T
        p = torch.exp(z - lse[:, None])
        inside = valid & (y >= c0) & (y < c0 + w.shape[0])
        rows = torch.nonzero(inside)[:, 0]
        p[rows, (y[rows] - c0)] -= 1.0
        p = p * (valid.to(dtype) / count)[:, None]
        dx += p @ w
        dw[c0:c0 + w.shape[0]] = p.T @ x
    return loss, dx.reshape(b, s, h), dw


def embedding_backward_reference(ids, grad, vocab, *, dtype=torch.float32):
    """``qwen3_triton/kernels/embedding.py:29-46``: dW[t] = sum of grad rows whose id is t."""
    h = grad.shape[-1]
    out = torch.zeros((vocab, h), dtype=dtype)
    out.index_add_(0, ids.reshape(-1), grad.reshape(-1, h).to(dtype))
    return out


# --------------------------------------------------------------------------- model
@dataclass
class OracleConfig:
    """Qwen3 architecture fields used by ``qwen3_triton/_model.py:60-108``."""
    vocab_size: int = 4096
    hidden_size: int = 256
    intermediate_size: int = 688
    num_hidden_layers: int = 4
    num_attention_heads: int = 8
    num_key_value_heads: int = 2
    head_dim: int = 32
    rope_theta: float = 1e6
    rms_norm_eps: float = 1e-6
    tie_word_embeddings: bool = False


def init_params(cfg, *, seed=0, std=0.02, dtype=torch.float32):
    """N(0,std) linear/embedding weights, norm weights 1 (``_model.py:34-48``), HF parameter names."""
    gen = torch.Generator().manual_seed(seed)

    def nrm(*shape):
        return (torch.randn(*shape, generator=gen) * std).to(dtype)

    h, d, i = cfg.hidden_size, cfg.head_dim, cfg.intermediate_size
    hq, hk = cfg.num_attention_heads, cfg.num_key_value_heads
    p = {"model.embed_tokens.weight": nrm(cfg.vocab_size, h)}
    for l in range(cfg.num_hidden_layers):
        pre = f"model.layers.{l}."
        p[pre + "self_attn.q_proj.weight"] = nrm(hq * d, h)
        p[pre + "self_attn.k_proj.weight"] = nrm(hk * d, h)
        p[pre + "self_attn.v_proj.weight"] = nrm(hk * d, h)
        p[pre + "self_attn.o_proj.weight"] = nrm(h, hq * d)
        p[pre + "self_attn.q_norm.weight"] = torch.ones(d, dtype=dtype)
        p[pre + "self_attn.k_norm.weight"] = torch.ones(d, dtype=dtype)
        p[pre + "mlp.gate_proj.weight"] = nrm(i, h)
        p[pre + "mlp.up_proj.weight"] = nrm(i, h)
        p[pre + "mlp.down_proj.weight"] = nrm(h, i)
        p[pre + "input_layernorm.weight"] = torch.ones(h, dtype=dtype)
        p[pre + "post_attention_layernorm.weight"] = torch.ones(h, dtype=dtype)
    p["model.norm.weight"] = torch.ones(h, dtype=dtype)
    p["lm_head.weight"] = p["model.embed_tokens.weight"] if cfg.tie_word_embeddings else nrm(cfg.vocab_size, h)
    return p


def decoder_layer_reference(x, p, pre, cfg, cos, sin, *, start=0, cache=None, dtype=torch.float32,
                            rounding=None):
    """One decoder layer, ``qwen3_triton/_model.py:60-91``.

    x [B,S,H]; cos/sin [B,S,D].  With ``cache`` (a dict holding fp K/V [B,Hk,L,D]) the new K/V are
    appended at ``start`` and attention runs over the whole prefix (``inference/model.py:114-119``).

    ``rounding`` (e.g. ``torch.bfloat16``) rounds every op's output to that type while the math
    stays in ``dtype``: the storage points of the reference's bf16 inference forward
    (``inference/model.py:108-137``: each kernel computes in fp32 and stores bf16 -- the input norm,
    the q/k/v projections, QK-norm + RoPE, attention, the o projection, the residual sum, the
    post-attention norm, gate and up, SwiGLU, the down projection, the residual sum).
    """
    b, s, h = x.shape
    d, hq, hk, eps = cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.rms_norm_eps
    W = lambda n: p[pre + n].to(dtype)  # noqa: E731
    R = (lambda t: t) if rounding is None else (lambda t: t.to(rounding).to(dtype))  # noqa: E731
    hn = R(rms_norm_reference(x, W("input_layernorm.weight"), eps, dtype=dtype))
    q = R(hn @ W("self_attn.q_proj.weight").T).view(b, s, hq, d)
    k = R(hn @ W("self_attn.k_proj.weight").T).view(b, s, hk, d)
    v = R(hn @ W("self_attn.v_proj.weight").T).view(b, s, hk, d)
    q, k = fused_qk_norm_rope_reference(q, k, W("self_attn.q_norm.weight"), W("self_attn.k_norm.weight"),
                                        cos, sin, eps, dtype=dtype)
    q, k, v = R(q).transpose(1, 2), R(k).transpose(1, 2), v.transpose(1, 2)
    if cache is not None:
        cache["k"] = k if cache.get("k") is None else torch.cat([cache["k"], k], dim=2)
        cache["v"] = v if cache.get("v") is None else torch.cat([cache["v"], v], dim=2)
        k, v = cache["k"], cache["v"]
    y = R(scaled_dot_product_attention_reference(q, k, v, scale=d ** -0.5, dtype=dtype))
    x = R(x.to(dtype) + R(y.transpose(1, 2).reshape(b, s, hq * d) @ W("self_attn.o_proj.weight").T))
    hn = R(rms_norm_reference(x, W("post_attention_layernorm.weight"), eps, dtype=dtype))
    m = R(swiglu_reference(hn @ W("mlp.gate_proj.weight").T, hn @ W("mlp.up_proj.weight").T, dtype=dtype))
    return R(x + R(m @ W("mlp.down_proj.weight").T))


def model_forward_reference(ids, p, cfg, *, labels=None, dtype=torch.float32, positions=None):
    """``qwen3_triton/_model.py:99-108,127-134``: embed, rope tables, layers, norm, lm_head, causal CE."""
    b, s = ids.shape
    x = p["model.embed_tokens.weight"].to(dtype)[ids]
    pos = torch.arange(s)[None, :].expand(b, s) if positions is None else positions
    cos, sin = rotary_tables_reference(pos, rope_inv_freq(cfg.rope_theta, cfg.head_dim), dtype=dtype)
    for l in range(cfg.num_hidden_layers):
        x = decoder_layer_reference(x, p, f"model.layers.{l}.", cfg, cos, sin, dtype=dtype)
    x = rms_norm_reference(x, p["model.norm.weight"], cfg.rms_norm_eps, dtype=dtype)
    logits = x @ p["lm_head.weight"].to(dtype).T
    loss = causal_cross_entropy_reference(logits, labels, dtype=dtype) if labels is not None else None
    return logits, loss


def argmax_lowest_reference(x):
    """``qwen3_triton/inference/kernels.py:150-161``: max value, lowest index among ties (NaN-free input)."""
    best = x.max(dim=-1, keepdim=True).values
    idx = torch.arange(x.shape[-1]).expand_as(x)
    return torch.where(x == best, idx, x.shape[-1]).min(dim=-1).values


def greedy_generate_reference(ids, p, cfg, max_new_tokens, *, eos=(), pad=0, dtype=torch.float32):
    """``qwen3_triton/inference/model.py:158-188`` with full recomputation each step (the
    ``use_cache=False`` verification mode of ``:149-151``).  Returns (tokens, top-2 margins)."""
    b, s = ids.shape
    out = ids.clone()
    done = torch.zeros(b, dtype=torch.bool)
    margins = []
    for step in range(max_new_tokens):
        logits, _ = model_forward_reference(out, p, cfg, dtype=dtype)
        last = logits[:, -1, :]
        tok = argmax_lowest_reference(last)
        top2 = last.topk(2, dim=-1).values
        margins.append((top2[:, 0] - top2[:, 1]))
        tok = torch.where(done, torch.full_like(tok, pad), tok)
        done = done | torch.isin(tok, torch.tensor(list(eos), dtype=tok.dtype)) if eos else done
        out = torch.cat([out, tok[:, None]], dim=1)
        if eos and bool(done.all()):
            break
    return out, torch.stack(margins, dim=1) if margins else torch.zeros(b, 0)


def cached_decode_reference(prompt, p, cfg, steps, *, forced=None, dtype=torch.float32):
    """Prefill + one-token-at-a-time decode through a K/V cache, ``inference/model.py:102-142,158-188``
    (``_forward`` with ``cache.length`` as the RoPE / causal offset, ``logits_to_keep=1``).

    The cache holds the already normed + rotated K and V of every position, so each step costs one
    token's matrix products instead of a full recomputation.  ``forced`` [B, steps] (optional)
    feeds fixed tokens instead of the greedy ones (teacher forcing), so a run can be compared step
    by step with another run's logits.  Returns (greedy tokens [B, steps] chosen after each of the
    ``steps`` forwards, last-position logits [B, steps, V]).  ``p`` should already be in ``dtype``
    (converting a 150K-row embedding per call is slow); norm weights may be any dtype.
    """
    b, s = prompt.shape
    caches = [dict() for _ in range(cfg.num_hidden_layers)]
    inv = rope_inv_freq(cfg.rope_theta, cfg.head_dim)
    emb = p["model.embed_tokens.weight"].to(dtype)
    head = p["lm_head.weight"].to(dtype)
    toks, logits_out = [], []
    cur, start = prompt, 0
    for step in range(steps):
        n = cur.shape[1]
        pos = torch.arange(start, start + n)[None, :].expand(b, n)
        cos, sin = rotary_tables_reference(pos, inv, dtype=dtype)
        x = emb[cur]
        for l in range(cfg.num_hidden_layers):
            x = decoder_layer_reference(x, p, f"model.layers.{l}.", cfg, cos, sin, start=start,
                                        cache=caches[l], dtype=dtype)
        x = rms_norm_reference(x[:, -1:], p["model.norm.weight"], cfg.rms_norm_eps, dtype=dtype)
        last = (x @ head.T)[:, 0]
        tok = argmax_lowest_reference(last)
        toks.append(tok)
        logits_out.append(last)
        start += n
        cur = (tok if forced is None else forced[:, step])[:, None]
    return torch.stack(toks, dim=1), torch.stack(logits_out, dim=1)
