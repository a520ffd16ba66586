"""Fused LM head + causal cross-entropy without materialising full fp32 logits.

New in this build (the reference materialises [B,S,V] logits: ``qwen3_triton/_model.py:131-132``
``lm_head`` then ``kernels/loss.py:46-71``).  The vocabulary is processed in chunks of ``chunk``
columns: each chunk's fp32 logits come from the matrix-core GEMM (h . W_c^T) into one reusable
[T, chunk] buffer and are folded into per-row (max, sum-exp) partials plus the target logit; a
final merge gives lse and the token-mean loss.  On the matrix-core path the logits GEMM's epilogue also
keeps each chunk's logits in the activation dtype (bf16: the reference's own lm_head output, whose
[T, V] copy it materialises too), and the statistics are formed from those stored values; the backward
turns them in place into dz = (softmax - onehot) * up / count plus dz^T, writes dW_c = dz_c^T . h per
chunk and dX = dz . W in one GEMM.  Other shapes recompute each chunk's logits in the backward.  The
same math as ``linear`` followed by ``causal_cross_entropy``.
"""
import torch

from . import _ops
from .linear import gemm_nt_into, matmul_into

DEFAULT_CHUNK = 16384


def _mfma_ok(x, w):
    return x.dtype in (torch.bfloat16, torch.float16) and x.shape[-1] % 8 == 0 and w.shape[0] % 8 == 0


def _chunk_logits(x, w, c0, n, zbuf):
    """zbuf[:, :n] = x . w[c0:c0+n]^T in fp32."""
    t, h = x.shape
    if _mfma_ok(x, w):
        gemm_nt_into(x, h, w[c0:c0 + n], h, zbuf, t, n, h)
    else:
        matmul_into(x, w[c0:c0 + n].t(), zbuf[:, :n])


class _LMHeadCE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, weight, labels, ignore_index, chunk):
        if not hidden.is_cuda or hidden.ndim != 3 or weight.ndim != 2 or weight.shape[1] != hidden.shape[-1]:
            raise ValueError('ROCm hidden [B,S,H] and weight [V,H] required')
        if labels.shape != hidden.shape[:2] or labels.dtype != torch.int64 or labels.device != hidden.device:
            raise ValueError('int64 [B,S] labels on the hidden device required')
        if hidden.dtype != weight.dtype or not hidden.is_contiguous() or not weight.is_contiguous():
            raise ValueError('Contiguous hidden/weight of one dtype required')
        b, s, h = hidden.shape
        v = weight.shape[0]
        if s < 2:
            raise ValueError('At least 2 tokens required')
        x = hidden.view(b * s, h)
        tgt = _ops.ce_shift_labels(labels, ignore_index)
        chunk = min(chunk, v)
        nch = -(-v // chunk)
        z = None
        if _mfma_ok(hidden, weight) and h % 64 == 0:
            # logits GEMM with the statistics epilogue: one partial per 128 logit columns, no fp32
            # logits in memory.  Where the shapes allow, the epilogue also keeps the logits in the
            # activation dtype (the reference's bf16 lm_head output) for the backward, which then
            # needs no second logits GEMM.
            groups = [-(-min(chunk, v - c * chunk) // 128) for c in range(nch)]
            st = _ops.CEState(b * s, sum(groups), hidden.device)
            if (b * s) % 8 == 0 and chunk % 8 == 0:
                z = torch.empty((b * s, -(-v // 64) * 64), device=hidden.device, dtype=hidden.dtype)
            part0 = 0
            for c in range(nch):
                c0 = c * chunk
                if z is not None:
                    st.gemm_stats_store(part0, x, weight, c0, min(chunk, v - c0), tgt, z[:, c0:])
                else:
                    st.gemm_stats(part0, x, weight, c0, min(chunk, v - c0), tgt)
                part0 += groups[c]
        else:
            st = _ops.CEState(b * s, nch, hidden.device)
            zbuf = torch.empty((b * s, chunk), device=hidden.device, dtype=torch.float32)
            for c in range(nch):
                c0 = c * chunk
                n = min(chunk, v - c0)
                _chunk_logits(x, weight, c0, n, zbuf)
                st.stats(c, zbuf, chunk, n, c0, tgt)
        loss = st.finish(tgt, v, ignore_index)
        ctx.save_for_backward(hidden, weight, tgt, st.lse, st.count)
        ctx.ignore, ctx.chunk = ignore_index, chunk
        ctx.z = z
        return loss.clone()

    @staticmethod
    def backward(ctx, dy):
        hidden, weight, tgt, lse, count = ctx.saved_tensors
        b, s, h = hidden.shape
        v, t, chunk = weight.shape[0], b * s, ctx.chunk
        x = hidden.view(t, h)
        up = dy.float().contiguous()
        dw = torch.empty_like(weight)
        mfma = _mfma_ok(x, weight) and t % 8 == 0
        z, ctx.z = ctx.z, None   # consumed: dz overwrites the stored logits in place
        if z is not None:
            # dz of every chunk from the stored logits, in place, and its transpose (the dW operand);
            # dW_c = dz_c^T . x per chunk, dX = dz . W in one GEMM over the whole vocabulary.
            vp = z.shape[1]
            if vp > v:
                z[:, v:].zero_()
            wt = _ops.transpose_last2(weight, pad_to=64)  # [H, Vp]
            xt = _ops.transpose_last2(x)                  # [H, T]
            dzt = torch.empty((chunk, t), device=x.device, dtype=x.dtype)
            for c in range(-(-v // chunk)):
                c0 = c * chunk
                n = min(chunk, v - c0)
                _ops.ce_grad_t(z[:, c0:], n, c0, tgt, lse, count, up, z[:, c0:], dzt, v, ctx.ignore)
                gemm_nt_into(dzt, t, xt, t, dw[c0:c0 + n], n, h, t)
            dx = torch.empty((t, h), device=x.device, dtype=x.dtype)
            gemm_nt_into(z, vp, wt, vp, dx, t, h, vp)
            return dx.view(b, s, h), dw, None, None, None
        if mfma and h % 64 == 0:
            # Every chunk's dz lands in one [T, Vp] buffer (Vp = V rounded up to 64, zero pad) written
            # by the logits GEMM's CE-gradient epilogue; dW_c = dz_c^T . x per chunk, and dX = dz . W
            # in one GEMM over the whole vocabulary at the end (bf16 out, no fp32 accumulation passes).
            vp = -(-v // 64) * 64
            wt = _ops.transpose_last2(weight, pad_to=64)  # [H, Vp]
            xt = _ops.transpose_last2(x)                  # [H, T]
            dz = torch.empty((t, vp), device=x.device, dtype=x.dtype)
            if vp > v:
                dz[:, v:].zero_()
            dzt = torch.empty((chunk, t), device=x.device, dtype=x.dtype)
            for c in range(-(-v // chunk)):
                c0 = c * chunk
                n = min(chunk, v - c0)
                dzc = dz[:, c0:c0 + n]
                if _ops.ce_grad_transposed_ok(x, t, n, vp, dzc, dzt):
                    # the CE-gradient GEMM stores dz and its transpose (the dW operand) itself
                    _ops.gemm_ce_grad(x, weight, c0, n, tgt, lse, count, up, dzc, v, ctx.ignore, dzt=dzt[:n])
                else:
                    _ops.gemm_ce_grad(x, weight, c0, n, tgt, lse, count, up, dzc, v, ctx.ignore)
                    _ops.transpose_into(dzc, dzt[:n])
                gemm_nt_into(dzt, t, xt, t, dw[c0:c0 + n], n, h, t)
            dx = torch.empty((t, h), device=x.device, dtype=x.dtype)
            gemm_nt_into(dz, vp, wt, vp, dx, t, h, vp)
            return dx.view(b, s, h), dw, None, None, None
        zbuf = torch.empty((t, chunk), device=x.device, dtype=torch.float32)
        dz = torch.empty((t, chunk), device=x.device, dtype=x.dtype)
        dx = torch.empty((t, h), device=x.device, dtype=torch.float32)
        if mfma:
            wt = _ops.transpose_last2(weight, pad_to=8)   # [H, Vp]
            xt = _ops.transpose_last2(x)                  # [H, T]
        for c in range(-(-v // chunk)):
            c0 = c * chunk
            n = min(chunk, v - c0)
            _chunk_logits(x, weight, c0, n, zbuf)
            _ops.ce_grad(zbuf, chunk, n, c0, tgt, lse, count, up, dz, chunk, v, ctx.ignore)
            if mfma:
                gemm_nt_into(dz, chunk, wt[:, c0:], wt.shape[1], dx, t, h, n, accumulate=c > 0)
                dzt = _ops.transpose_last2(dz)            # [chunk, T]
                gemm_nt_into(dzt, t, xt, t, dw[c0:c0 + n], n, h, t)
            else:
                matmul_into(dz[:, :n], weight[c0:c0 + n], dx, accumulate=c > 0)
                matmul_into(dz[:, :n].t(), x, dw[c0:c0 + n])
        return _ops.cast(dx, x.dtype).view(b, s, h), dw, None, None, None


def lm_head_cross_entropy(hidden, weight, labels, *, ignore_index=-100, chunk=DEFAULT_CHUNK):
    """Causal token-mean CE of ``hidden @ weight.T`` against ``labels`` (shift inside), fused."""
    return _LMHeadCE.apply(hidden, weight, labels, ignore_index, chunk)
