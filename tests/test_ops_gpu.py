"""HIP bandwidth-bound ops vs the CPU oracle (bf16/fp16 forward: max-rel <= 2e-2 / 3e-3; gradients:
cosine >= 0.999 and max-rel <= the same bounds; fp32: 1e-5)."""
import pytest
import torch

import oracle as O
from _util import cosine, max_rel, randn, seeded, tol_for

from qwen3_triton.kernels import _ops
from qwen3_triton.kernels.norm import rms_norm, rms_norm_fork
from qwen3_triton.kernels.norm_rope import norm_rope
from qwen3_triton.kernels.rotary import apply_rotary, rotary_tables
from qwen3_triton.kernels.activation import swiglu
from qwen3_triton.kernels.residual import residual_add
from qwen3_triton.kernels.embedding import embedding
from ops.triton.rms_norm import rms_norm_triton
from ops.triton.rope import apply_rope_triton
from ops.triton.fused_qk_norm_rope import fused_qk_norm_rope_triton
from ops.triton.silu_and_mul import silu_and_mul_triton

pytestmark = pytest.mark.gpu
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _grads(out, inputs, up):
    return torch.autograd.grad(out, inputs, up)


def check(actual, expected, dtype, what):
    tol = tol_for(dtype) * (2 if dtype == torch.float32 else 1)
    r = max_rel(actual, expected)
    assert r <= tol, f"{what}: max-rel {r:.3e} > {tol}"
    if expected.numel() > 1 and expected.double().abs().max() > 0:
        c = cosine(actual, expected)
        assert c >= 0.999, f"{what}: cosine {c:.6f}"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(2, 7, 128), (1, 17, 2048), (3, 4096), (5, 24), (2, 3, 5120), (2, 8192),
                                   (1, 1, 128), (64, 256)])
def test_rmsnorm_fwd_bwd(shape, dtype):
    print(f"rmsnorm {shape} {dtype}", flush=True)
    gen = seeded(1)
    h = shape[-1]
    x = randn(*shape, gen=gen, dtype=dtype)
    w = randn(h, gen=gen, dtype=dtype, scale=0.1, shift=1.0)
    dy = randn(*shape, gen=gen, dtype=dtype)
    xd, wd = x.cuda().requires_grad_(), w.cuda().requires_grad_()
    y = rms_norm(xd, wd, 1e-6)
    dx, dw = _grads(y, (xd, wd), dy.cuda())
    check(y, O.rms_norm_reference(x, w, 1e-6), dtype, "y")
    ex, ew = O.rms_norm_backward_reference(x, w, dy, 1e-6)
    check(dx, ex, dtype, "dx")
    check(dw, ew, dtype, "dw")
    # deterministic: same inputs, bitwise-equal weight gradient
    _, dw2 = _grads(rms_norm(xd, wd, 1e-6), (xd, wd), dy.cuda())
    assert torch.equal(dw, dw2)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(2, 7, 128), (3, 4096), (5, 24), (2, 3, 5120), (2, 8192), (1, 1, 10000)])
def test_rmsnorm_fork_residual_gradient(shape, dtype):
    """x -> (x, rms_norm(x)) feeding x + f(norm(x)): dx = g + norm_bwd(g * df) from one kernel
    (q3_rmsnorm_bwd_add, the scalar path with its add for h = 10000), against the oracle."""
    print(f"rmsnorm fork {shape} {dtype}", flush=True)
    gen = seeded(3)
    h = shape[-1]
    x = randn(*shape, gen=gen, dtype=dtype)
    w = randn(h, gen=gen, dtype=dtype, scale=0.1, shift=1.0)
    g = randn(*shape, gen=gen, dtype=dtype)
    c = randn(*shape, gen=gen, dtype=dtype)   # y = x + c * norm(x): the norm branch's upstream grad is g * c
    xd, wd, cd = x.cuda().requires_grad_(), w.cuda().requires_grad_(), c.cuda()
    xa, n = rms_norm_fork(xd, wd, 1e-6)
    assert xa.data_ptr() == xd.data_ptr()
    y = residual_add(xa, (n.float() * cd.float()).to(dtype))
    dx, dw = _grads(y, (xd, wd), g.cuda())
    gn = (g.double() * c.double()).to(dtype)
    ex, ew = O.rms_norm_backward_reference(x, w, gn, 1e-6)
    check(dx, (g.double() + ex.double()).to(dtype), dtype, "dx")
    check(dw, ew, dtype, "dw")
    # the fused kernel equals norm backward + residual add, bit for bit on the same inputs
    dx1, dw1 = _ops.rmsnorm_bwd(xd.detach(), wd.detach(), gn.cuda(), 1e-6)
    dx2, dw2 = _ops.rmsnorm_bwd_add(xd.detach(), wd.detach(), gn.cuda(), g.cuda(), 1e-6)
    assert torch.equal(dw1, dw2)
    assert torch.equal(_ops.add(dx1, g.cuda()), dx2)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("b,s,hq,hk,d", [(2, 5, 4, 2, 128), (1, 17, 32, 8, 128), (2, 3, 4, 2, 64),
                                         (1, 4, 2, 1, 24), (1, 3, 2, 2, 256)])
def test_norm_rope_fwd_bwd(b, s, hq, hk, d, dtype):
    print(f"norm_rope {b} {s} {hq} {hk} {d} {dtype}", flush=True)
    gen = seeded(2)
    q = randn(b, s, hq, d, gen=gen, dtype=dtype)
    k = randn(b, s, hk, d, gen=gen, dtype=dtype)
    qw = randn(d, gen=gen, dtype=dtype, scale=0.1, shift=1.0)
    kw = randn(d, gen=gen, dtype=dtype, scale=0.1, shift=1.0)
    # independent random tables (not real angles) exercise the general transpose
    c = randn(b, s, d, gen=gen, dtype=dtype)
    sn = randn(b, s, d, gen=gen, dtype=dtype)
    gq = randn(b, s, hq, d, gen=gen, dtype=dtype)
    gk = randn(b, s, hk, d, gen=gen, dtype=dtype)
    dev = [t.cuda() for t in (q, k, qw, kw)]
    for t in dev:
        t.requires_grad_()
    yq, yk = fused_qk_norm_rope_triton(*dev, c.cuda(), sn.cuda(), 1e-6)
    grads = _grads((yq, yk), dev, (gq.cuda(), gk.cuda()))
    eq, ek = O.fused_qk_norm_rope_reference(q, k, qw, kw, c, sn, 1e-6)
    check(yq, eq, dtype, "yq")
    check(yk, ek, dtype, "yk")
    e = O.fused_qk_norm_rope_backward_reference(q, k, qw, kw, c, sn, gq, gk, 1e-6)
    for a, x, n in zip(grads, e, ("dq", "dk", "dqw", "dkw")):
        check(a, x, dtype, n)
    # the single-tensor module API (kernels/norm_rope.py) agrees with the pair API
    y1 = norm_rope(dev[0].detach(), dev[2].detach(), c.cuda(), sn.cuda(), 1e-6)
    assert torch.equal(y1, yq.detach())
    # fp32 weights and tables beside 16-bit activations (the reference reads every operand as fp32)
    if dtype != torch.float32:
        c32, s32 = randn(b, s, d, gen=gen, dtype=torch.float32), randn(b, s, d, gen=gen, dtype=torch.float32)
        w32 = [randn(d, gen=gen, dtype=torch.float32, scale=0.1, shift=1.0) for _ in range(2)]
        dm = [q.cuda().requires_grad_(), k.cuda().requires_grad_()] + [w.cuda().requires_grad_() for w in w32]
        yq, yk = fused_qk_norm_rope_triton(*dm, c32.cuda(), s32.cuda(), 1e-6)
        assert yq.dtype == dtype and yk.dtype == dtype
        grads = _grads((yq, yk), dm, (gq.cuda(), gk.cuda()))
        assert grads[0].dtype == dtype and grads[2].dtype == torch.float32
        eq, ek = O.fused_qk_norm_rope_reference(q.float(), k.float(), *w32, c32, s32, 1e-6)
        check(yq, eq, dtype, "yq[mixed]")
        check(yk, ek, dtype, "yk[mixed]")
        e = O.fused_qk_norm_rope_backward_reference(q.float(), k.float(), *w32, c32, s32, gq.float(), gk.float(),
                                                    1e-6)
        for a, x, n in zip(grads, e, ("dq", "dk", "dqw", "dkw")):
            check(a, x, dtype, n + "[mixed]")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("b,s,h,d", [(2, 7, 4, 16), (1, 129, 2, 128), (2, 3, 3, 6)])
def test_rope_both_layouts(b, s, h, d, dtype):
    print(f"rope {b} {s} {h} {d} {dtype}", flush=True)
    gen = seeded(3)
    x = randn(b, s, h, d, gen=gen, dtype=dtype)
    c = randn(b, s, d, gen=gen, dtype=dtype)
    sn = randn(b, s, d, gen=gen, dtype=dtype)
    gy = randn(b, s, h, d, gen=gen, dtype=dtype)
    xd = x.cuda().requires_grad_()
    y = apply_rotary(xd, c.cuda(), sn.cuda())
    (dx,) = _grads(y, (xd,), gy.cuda())
    e, _ = O.apply_rope_reference(x.transpose(1, 2), x.transpose(1, 2), c, sn)
    check(y, e.transpose(1, 2), dtype, "y")
    eg, _ = O.apply_rope_backward_reference(gy.transpose(1, 2), gy.transpose(1, 2), c, sn)
    check(dx, eg.transpose(1, 2), dtype, "dx")
    # [B,H,S,D] layout through ops.triton
    xh = x.transpose(1, 2).contiguous().cuda().requires_grad_()
    yq, yk = apply_rope_triton(xh, xh, c.cuda(), sn.cuda())
    check(yq, e, dtype, "yq[BHSD]")
    (dxh,) = _grads(yq, (xh,), gy.transpose(1, 2).contiguous().cuda())
    check(dxh, eg, dtype, "dx[BHSD]")
    # fp32 tables beside 16-bit activations, as the reference's kernel accepts them
    if dtype != torch.float32:
        c32 = randn(b, s, d, gen=gen, dtype=torch.float32)
        s32 = randn(b, s, d, gen=gen, dtype=torch.float32)
        xm = x.transpose(1, 2).contiguous().cuda().requires_grad_()
        ym, _ = apply_rope_triton(xm, xm.detach(), c32.cuda(), s32.cuda())
        assert ym.dtype == dtype
        em, _ = O.apply_rope_reference(x.transpose(1, 2).float(), x.transpose(1, 2).float(), c32, s32)
        check(ym, em, dtype, "yq[fp32 tables]")
        (dxm,) = _grads(ym, (xm,), gy.transpose(1, 2).contiguous().cuda())
        egm, _ = O.apply_rope_backward_reference(gy.transpose(1, 2).float(), gy.transpose(1, 2).float(), c32, s32)
        check(dxm, egm, dtype, "dx[fp32 tables]")


@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_tables_against_oracle(dtype):
    pos = torch.arange(2048).repeat(2).view(2, 2048)
    inv = O.rope_inv_freq(1e6, 128)
    c, s = rotary_tables(pos.cuda(), inv.cuda(), dtype)
    ec, es = O.rotary_tables_reference(pos, inv)
    tol = {torch.float32: 2e-6, torch.float16: 1e-3, torch.bfloat16: 8e-3}[dtype]
    assert (c.float().cpu() - ec).abs().max() <= tol
    assert (s.float().cpu() - es).abs().max() <= tol
    c32, _ = rotary_tables(pos.int().cuda(), inv.cuda(), dtype)
    assert torch.equal(c32, c)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(1, 1), (2, 17), (1, 129, 257), (3, 6144), (4099,)])
def test_swiglu_fwd_bwd(shape, dtype):
    print(f"swiglu {shape} {dtype}", flush=True)
    gen = seeded(4)
    gt = randn(*shape, gen=gen, dtype=dtype)
    ut = randn(*shape, gen=gen, dtype=dtype)
    dy = randn(*shape, gen=gen, dtype=dtype)
    gd, ud = gt.cuda().requires_grad_(), ut.cuda().requires_grad_()
    y = silu_and_mul_triton(gd, ud)
    dg, du = _grads(y, (gd, ud), dy.cuda())
    check(y, O.swiglu_reference(gt, ut), dtype, "y")
    eg, eu = O.swiglu_backward_reference(gt, ut, dy)
    check(dg, eg, dtype, "dg")
    check(du, eu, dtype, "du")
    assert torch.equal(swiglu(gd.detach(), ud.detach()), y.detach())


@pytest.mark.parametrize("dtype", DTYPES)
def test_residual_cast_fill_transpose(dtype):
    gen = seeded(5)
    a = randn(3, 1000, gen=gen, dtype=dtype)
    b = randn(3, 1000, gen=gen, dtype=dtype)
    c = residual_add(a.cuda(), b.cuda())
    assert torch.equal(c.cpu(), (a.float() + b.float()).to(dtype))
    x = randn(2, 67, 130, gen=gen, dtype=dtype)
    assert torch.equal(_ops.transpose_last2(x.cuda()).cpu(), x.transpose(1, 2).contiguous())
    y = _ops.cast(x.cuda(), torch.float32)
    assert torch.equal(y.cpu(), x.float())
    z = _ops.fill_(torch.empty(1001, device="cuda", dtype=dtype), 1.5)
    assert bool((z == 1.5).all())
    p = _ops.positions(2, 5, 7, "cuda")
    assert p.cpu().tolist() == [[7, 8, 9, 10, 11]] * 2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("r,c", [(64, 256), (8192, 1024), (384, 128), (72, 40), (37, 50)])
def test_strided_data_movement(r, c, dtype):
    """q3_transpose2d into a column block of a wider matrix writes nothing else; q3_copy2d and the
    row-strided SwiGLU backward match their contiguous forms bit for bit."""
    gen = seeded(r + c)
    x = torch.randn(r, c, generator=gen).to(dtype).cuda()
    wide = torch.full((c, 3 * r), 7.0, dtype=dtype, device="cuda")
    _ops.transpose_into(x, wide[:, r:2 * r])
    assert torch.equal(wide[:, r:2 * r].cpu(), x.t().cpu())
    assert bool((wide[:, :r] == 7).all()) and bool((wide[:, 2 * r:] == 7).all())
    dst = torch.full((r, 2 * c), 5.0, dtype=dtype, device="cuda")
    _ops.copy_into(x, dst[:, c:])
    assert torch.equal(dst[:, c:].cpu(), x.cpu()) and bool((dst[:, :c] == 5).all())
    g, u, dy = (torch.randn(r, c, generator=gen).to(dtype).cuda() for _ in range(3))
    eg, eu = _ops.swiglu_bwd(g, u, dy)
    both = torch.empty(r, 2 * c, dtype=dtype, device="cuda")
    _ops.swiglu_bwd_into(g, u, dy, both[:, :c], both[:, c:])
    assert torch.equal(both[:, :c].cpu(), eg.cpu()) and torch.equal(both[:, c:].cpu(), eu.cpu())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("batch,r,c,pad", [(1, 8192, 4096, 1), (2, 67, 136, 8), (1, 70, 264, 64), (3, 5, 8, 16),
                                           (1, 2048, 1024, 8), (2, 67, 130, 1), (3, 256, 384, 1), (2, 128, 256, 64)])
def test_transpose_shapes(batch, r, c, pad, dtype):
    """Bit-exact layout change, vector (cols % 8 == 0, padded ld % 8 == 0) and scalar paths; the pad
    columns are zero."""
    print(f"transpose {batch}x{r}x{c} pad {pad} {dtype}", flush=True)
    x = torch.randn(batch, r, c, generator=seeded(r + c), dtype=torch.float32).to(dtype)
    y = _ops.transpose_last2(x.cuda(), pad_to=pad).cpu()
    rp = -(-r // pad) * pad
    assert y.shape == (batch, c, rp)
    assert torch.equal(y[..., :r], x.transpose(1, 2))
    assert not bool(y[..., r:].any())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("h", [64, 4096, 12])
def test_embedding_fwd_bwd_deterministic(h, dtype):
    gen = seeded(6)
    v = 50
    w = randn(v, h, gen=gen, dtype=dtype)
    ids = torch.randint(0, v, (3, 40), generator=gen)
    ids[0, :5] = 7  # repeated ids
    dy = randn(3, 40, h, gen=gen, dtype=dtype)
    wd = w.cuda().requires_grad_()
    y = embedding(ids.cuda(), wd)
    assert torch.equal(y.detach().cpu(), w[ids])
    (dw,) = _grads(y, (wd,), dy.cuda())
    check(dw, O.embedding_backward_reference(ids, dy, v), dtype, "dw")
    (dw2,) = _grads(embedding(ids.int().cuda(), wd), (wd,), dy.cuda())
    assert torch.equal(dw, dw2)


def test_embedding_out_of_range_raises():
    w = torch.randn(10, 8, device="cuda")
    with pytest.raises(ValueError):
        embedding(torch.tensor([[1, 10]], device="cuda"), w)


def test_norm_rope_pair_validates_like_norm_rope():
    """The Q/K pair op applies the single-tensor op's checks to both tensors: a weight or table in
    another dtype than the activations, or a rotary table that requires grad, is rejected."""
    from qwen3_triton.kernels.norm_rope import norm_rope_pair
    q = torch.randn(1, 4, 8, 128, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(1, 4, 2, 128, device="cuda", dtype=torch.bfloat16)
    w = torch.ones(128, device="cuda", dtype=torch.bfloat16)
    cos = torch.ones(1, 4, 128, device="cuda", dtype=torch.bfloat16)
    sin = torch.zeros(1, 4, 128, device="cuda", dtype=torch.bfloat16)
    norm_rope_pair(q, k, w, w, cos, sin)
    with pytest.raises(ValueError):
        norm_rope_pair(q, k, w.float(), w, cos, sin)
    with pytest.raises(ValueError):
        norm_rope_pair(q, k, w, w.float(), cos, sin)
    with pytest.raises(ValueError):
        norm_rope_pair(q, k, w, w, cos.float(), sin.float())
    with pytest.raises(ValueError):
        norm_rope_pair(q, k, w, w, cos.clone().requires_grad_(), sin)


@pytest.mark.gpu
def test_module_validation_matches_reference():
    """Argument checks that raise before any launch, as ``kernels/norm.py:47``, ``embedding.py:59``
    and ``norm_rope.py:57`` raise them."""
    from qwen3_triton.kernels.embedding import embedding
    x = torch.randn(2, 8200, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="H<=8192"):
        rms_norm(x, torch.ones(8200, device="cuda", dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="positive epsilon"):
        rms_norm(x[:, :64].contiguous(), torch.ones(64, device="cuda", dtype=torch.bfloat16), 0.0)
    ids = torch.zeros(4, dtype=torch.int64, device="cuda")
    with pytest.raises(ValueError, match="Nonempty vocabulary"):
        embedding(ids, torch.empty(0, 8, device="cuda", dtype=torch.bfloat16))
    q = torch.zeros(1, 2, 2, 8, device="cuda", dtype=torch.int32)
    cs = torch.zeros(1, 2, 8, device="cuda", dtype=torch.int32)
    with pytest.raises(ValueError, match="Floating point, even nonempty D"):
        norm_rope(q, torch.zeros(8, device="cuda", dtype=torch.int32), cs, cs, 1e-6)
    qo = torch.randn(1, 2, 2, 7, device="cuda", dtype=torch.bfloat16)
    co = torch.randn(1, 2, 7, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="Floating point, even nonempty D"):
        norm_rope(qo, torch.ones(7, device="cuda", dtype=torch.bfloat16), co, co, 1e-6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(3, 4096), (2, 20000)])
def test_rms_norm_triton_op(shape, dtype):
    """``ops/triton/rms_norm.py:118-138``: forward and backward against the oracle, including rows wider
    than the vector path (the scalar kernels); wider than 65536 is rejected as the reference rejects it."""
    print(f"rms_norm_triton {shape} {dtype}", flush=True)
    gen = seeded(5)
    h = shape[-1]
    x = randn(*shape, gen=gen, dtype=dtype)
    w = randn(h, gen=gen, dtype=dtype, scale=0.1, shift=1.0)
    dy = randn(*shape, gen=gen, dtype=dtype)
    xd, wd = x.cuda().requires_grad_(), w.cuda().requires_grad_()
    y = rms_norm_triton(xd, wd, 1e-6)
    dx, dw = _grads(y, (xd, wd), dy.cuda())
    check(y, O.rms_norm_reference(x, w, 1e-6), dtype, "y")
    ex, ew = O.rms_norm_backward_reference(x, w, dy, 1e-6)
    check(dx, ex, dtype, "dx")
    check(dw, ew, dtype, "dw")
    with pytest.raises(ValueError, match="too large"):
        rms_norm_triton(torch.ones(1, 65537, device="cuda", dtype=dtype), torch.ones(65537, device="cuda", dtype=dtype))
