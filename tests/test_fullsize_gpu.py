"""Config #2 at its benchmark shapes (seed 1): RMSNorm [8192 x 4096], per-head QK-norm + RoPE on
Q [8192 x 32 x 128] / K [8192 x 8 x 128] at positions 0..2047 repeated over batch 4, and SwiGLU
[8192 x 12288], forward and backward, against the fp32 oracle on the host.

These are the sizes ``bench.py`` times.  The streaming kernels size their grids from the data
(one pass over the rows), so this checks their grid and tail indexing where the small-shape tests
cannot.  Every output is checked normwise over the whole tensor (max-rel <= 2e-2, cosine >= 0.999)
and row by row (each row's max |error| <= 2e-2 of that row's max |expected|), so one missed or
misplaced row fails even when it is a tiny part of the tensor."""
import pytest
import torch

import oracle as O
from _util import cosine, max_rel, randn, seeded

from qwen3_triton.kernels.activation import swiglu
from qwen3_triton.kernels.norm import rms_norm
from qwen3_triton.kernels.norm_rope import norm_rope, norm_rope_pair
from qwen3_triton.kernels.rotary import rotary_tables

pytestmark = pytest.mark.gpu
T, H, HQ, HK, D, I = 8192, 4096, 32, 8, 128, 12288


def check(actual, expected, what, rows):
    a = actual.detach().float().cpu().reshape(rows, -1)
    e = expected.float().reshape(rows, -1)
    r = max_rel(a, e)
    c = cosine(a, e)
    row_err = (a - e).abs().amax(dim=1)
    row_ref = e.abs().amax(dim=1).clamp_min(1e-30)
    worst = float((row_err / row_ref).max())
    print(f"{what}: max-rel {r:.2e} cosine {c:.7f} worst row {worst:.2e}", flush=True)
    assert r <= 2e-2 and c >= 0.999, what
    assert worst <= 2e-2, f"{what}: row {int((row_err / row_ref).argmax())} off by {worst:.2e}"


def test_rmsnorm_8192x4096():
    gen = seeded(1)
    x = randn(T, H, gen=gen, dtype=torch.bfloat16)
    w = randn(H, gen=gen, dtype=torch.bfloat16, scale=0.1, shift=1.0)
    dy = randn(T, H, gen=gen, dtype=torch.bfloat16)
    xd, wd = x.cuda().requires_grad_(), w.cuda().requires_grad_()
    y = rms_norm(xd, wd, 1e-6)
    dx, dw = torch.autograd.grad(y, (xd, wd), dy.cuda())
    check(y, O.rms_norm_reference(x, w, 1e-6), "rmsnorm y", T)
    ex, ew = O.rms_norm_backward_reference(x, w, dy, 1e-6)
    check(dx, ex, "rmsnorm dx", T)
    check(dw, ew, "rmsnorm dw", 1)


@pytest.mark.parametrize("heads", [HQ, HK])
def test_qk_norm_rope_full_size(heads):
    gen = seeded(1)
    x = randn(4, 2048, heads, D, gen=gen, dtype=torch.bfloat16)
    w = randn(D, gen=gen, dtype=torch.bfloat16, scale=0.1, shift=1.0)
    dy = randn(4, 2048, heads, D, gen=gen, dtype=torch.bfloat16)
    pos = torch.arange(2048)[None].expand(4, 2048).contiguous()
    cos, sin = rotary_tables(pos.cuda(), O.rope_inv_freq(1e6, D).cuda(), torch.bfloat16)
    ec, es = O.rotary_tables_reference(pos, O.rope_inv_freq(1e6, D), dtype=torch.bfloat16)
    assert torch.equal(cos.cpu(), ec) or max_rel(cos, ec) <= 1e-2
    xd, wd = x.cuda().requires_grad_(), w.cuda().requires_grad_()
    y = norm_rope(xd, wd, cos, sin, 1e-6)
    dx, dw = torch.autograd.grad(y, (xd, wd), dy.cuda())
    cf, sf = cos.float().cpu(), sin.float().cpu()
    # one tensor through the pair oracle: pass it as both q and k and keep the q half
    ey, _ = O.fused_qk_norm_rope_reference(x, x[:, :, :1], w, w, cf, sf, 1e-6)
    check(y, ey, f"norm_rope[{heads}] y", T * heads)
    edx, _, edw, _ = O.fused_qk_norm_rope_backward_reference(x, x[:, :, :1], w, w, cf, sf, dy, dy[:, :, :1], 1e-6)
    check(dx, edx, f"norm_rope[{heads}] dx", T * heads)
    check(dw, edw, f"norm_rope[{heads}] dw", 1)


def test_qk_norm_rope_pair_full_size():
    """Q and K heads of the layer in one launch per direction: checked against the pair oracle row by
    row, and y / dx bit-identical to the single-tensor launches (same per-row arithmetic)."""
    gen = seeded(5)
    q = randn(4, 2048, HQ, D, gen=gen, dtype=torch.bfloat16)
    k = randn(4, 2048, HK, D, gen=gen, dtype=torch.bfloat16)
    wq = randn(D, gen=gen, dtype=torch.bfloat16, scale=0.1, shift=1.0)
    wk = randn(D, gen=gen, dtype=torch.bfloat16, scale=0.1, shift=1.0)
    gq = randn(4, 2048, HQ, D, gen=gen, dtype=torch.bfloat16)
    gk = randn(4, 2048, HK, D, gen=gen, dtype=torch.bfloat16)
    pos = torch.arange(2048)[None].expand(4, 2048).contiguous()
    cos, sin = rotary_tables(pos.cuda(), O.rope_inv_freq(1e6, D).cuda(), torch.bfloat16)
    dev = [t.cuda().requires_grad_() for t in (q, k, wq, wk)]
    yq, yk = norm_rope_pair(*dev, cos, sin, 1e-6)
    dq, dk, dwq, dwk = torch.autograd.grad((yq, yk), dev, (gq.cuda(), gk.cuda()))
    cf, sf = cos.float().cpu(), sin.float().cpu()
    eq, ek = O.fused_qk_norm_rope_reference(q, k, wq, wk, cf, sf, 1e-6)
    check(yq, eq, "pair yq", T * HQ)
    check(yk, ek, "pair yk", T * HK)
    edq, edk, edwq, edwk = O.fused_qk_norm_rope_backward_reference(q, k, wq, wk, cf, sf, gq, gk, 1e-6)
    check(dq, edq, "pair dq", T * HQ)
    check(dk, edk, "pair dk", T * HK)
    check(dwq, edwq, "pair dwq", 1)
    check(dwk, edwk, "pair dwk", 1)
    for x, w, y, g, dx in ((dev[0], dev[2], yq, gq, dq), (dev[1], dev[3], yk, gk, dk)):
        xs, ws = x.detach().clone().requires_grad_(), w.detach().clone().requires_grad_()
        ys = norm_rope(xs, ws, cos, sin, 1e-6)
        dxs, dws = torch.autograd.grad(ys, (xs, ws), g.cuda())
        assert torch.equal(ys, y.detach()) and torch.equal(dxs, dx)
        assert max_rel(dws, edwq if w is dev[2] else edwk) <= 2e-2


def test_swiglu_8192x12288():
    gen = seeded(1)
    g = randn(T, I, gen=gen, dtype=torch.bfloat16)
    u = randn(T, I, gen=gen, dtype=torch.bfloat16)
    dy = randn(T, I, gen=gen, dtype=torch.bfloat16)
    gd, ud = g.cuda().requires_grad_(), u.cuda().requires_grad_()
    y = swiglu(gd, ud)
    dg, du = torch.autograd.grad(y, (gd, ud), dy.cuda())
    check(y, O.swiglu_reference(g, u), "swiglu y", T)
    del y
    eg, eu = O.swiglu_backward_reference(g, u, dy)
    check(dg, eg, "swiglu dg", T)
    check(du, eu, "swiglu du", T)
