"""Matrix-core GEMM (q3_gemm_nt) and the strided fallback vs fp64 torch.matmul on the host."""
import pytest
import torch

from _util import cosine, max_rel, randn, seeded

from qwen3_triton.kernels.linear import gemm_nt_into, linear, matmul, matmul_into

pytestmark = pytest.mark.gpu


def ref(a, b):
    """fp64 product; the largest shapes run it on the device (rocBLAS dgemm) to keep the test short."""
    if a.shape[0] * a.shape[1] * b.shape[1] > 2 ** 36:
        return (a.cuda().double() @ b.cuda().double()).cpu()
    return (a.double() @ b.double())


@pytest.mark.parametrize("m,n,k", [(32, 32, 16), (256, 128, 64), (300, 200, 8), (1, 4096, 4096), (8, 1024, 4096),
                                   (513, 687, 688), (2048, 1024, 4096), (64, 151936 // 16, 256), (1000, 3000, 128),
                                   (8192, 4096, 4096), (4096, 12288, 640), (8192, 1024, 192), (333, 4100, 4160),
                                   (4353, 4100, 1024), (2050, 4000, 512), (6144, 4096, 256),
                                   (5000, 4096, 128), (3072, 4096, 256), (3000, 4000, 192),
                                   (4096, 12288, 8192), (6144, 4096, 8192)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_nt_shapes(m, n, k, dtype):
    print(f"gemm_nt {m}x{n}x{k} {dtype}", flush=True)
    gen = seeded(m * 7 + n + k)
    a = randn(m, k, gen=gen, dtype=dtype)
    w = randn(n, k, gen=gen, dtype=dtype)
    out = torch.empty(m, n, device="cuda", dtype=torch.float32)
    gemm_nt_into(a.cuda(), k, w.cuda(), k, out, m, n, k)
    e = ref(a, w.t())
    r = max_rel(out, e)
    assert r < 1e-5, r  # fp32 accumulation of exact bf16 products
    y = matmul(a.cuda(), w.cuda().t())
    assert y.dtype == dtype
    assert max_rel(y, e) < (8e-3 if dtype == torch.bfloat16 else 1e-3)


def test_gemm_alpha_accumulate_and_ldc():
    gen = seeded(9)
    a = randn(70, 64, gen=gen, dtype=torch.bfloat16)
    b = randn(90, 64, gen=gen, dtype=torch.bfloat16)
    c0 = randn(70, 100, gen=gen)
    out = c0.clone().cuda()
    gemm_nt_into(a.cuda(), 64, b.cuda(), 64, out, 70, 90, 64, alpha=0.5, accumulate=True)
    e = c0.double().clone()
    e[:, :90] += 0.5 * ref(a, b.t())
    assert max_rel(out, e) < 1e-5
    assert torch.equal(out[:, 90:].cpu(), c0[:, 90:])  # columns beyond N untouched


@pytest.mark.parametrize("m,n", [(4352, 4096), (4353, 4100), (2050, 4000)])
def test_gemm_persistent_accumulate(m, n):
    """More output tiles than CUs: workgroups stream several tiles (EVEN and edge-clamped paths)
    and accumulate into an fp32 output with a row pitch wider than N."""
    print(f"gemm_nt accumulate {m}x{n}", flush=True)
    gen = seeded(m + n)
    k = 256
    a = randn(m, k, gen=gen, dtype=torch.bfloat16)
    b = randn(n, k, gen=gen, dtype=torch.bfloat16)
    c0 = randn(m, n + 8, gen=gen)
    out = c0.clone().cuda()
    gemm_nt_into(a.cuda(), k, b.cuda(), k, out, m, n, k, alpha=2.0, accumulate=True)
    e = c0.double().clone()
    e[:, :n] += 2.0 * ref(a, b.t())
    assert max_rel(out, e) < 1e-5
    assert torch.equal(out[:, n:].cpu(), c0[:, n:])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_matmul_layouts(dtype):
    """NT direct, NN and TN (operands re-laid out by the transpose kernel), and fp32 (SIMT path)."""
    gen = seeded(10)
    x = randn(200, 96, gen=gen, dtype=dtype)
    w = randn(136, 96, gen=gen, dtype=dtype)
    dy = randn(200, 136, gen=gen, dtype=dtype)
    tol = 8e-3 if dtype == torch.bfloat16 else 1e-5
    xd, wd, dyd = x.cuda(), w.cuda(), dy.cuda()
    assert max_rel(matmul(xd, wd.t()), ref(x, w.t())) < tol
    assert max_rel(matmul(dyd, wd), ref(dy, w)) < tol
    assert max_rel(matmul(dyd.t(), xd), ref(dy.t(), x)) < tol
    assert max_rel(matmul(xd[:, ::2], wd[:, ::2].t()), ref(x[:, ::2], w[:, ::2].t())) < tol


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_linear_autograd(dtype):
    gen = seeded(11)
    x = randn(4, 33, 64, gen=gen, dtype=dtype)
    w = randn(80, 64, gen=gen, dtype=dtype, scale=0.1)
    dy = randn(4, 33, 80, gen=gen, dtype=dtype)
    xd, wd = x.cuda().requires_grad_(), w.cuda().requires_grad_()
    y = linear(xd, wd)
    dx, dw = torch.autograd.grad(y, (xd, wd), dy.cuda())
    xr, wr = x.double().requires_grad_(), w.double().requires_grad_()
    yr = xr @ wr.t()
    ex, ew = torch.autograd.grad(yr, (xr, wr), dy.double())
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    for a, e in ((y, yr), (dx, ex), (dw, ew)):
        assert max_rel(a, e) < tol
        assert cosine(a, e) > 0.999


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_shared_input_projections_autograd(dtype):
    """q/k/v-style projections sharing one input: outputs and all gradients against fp64 autograd
    (bf16 takes the packed single-GEMM backward, fp32 the per-projection path)."""
    from qwen3_triton.kernels.linear import shared_input_projections
    gen = seeded(12)
    x = randn(2, 40, 256, gen=gen, dtype=dtype)
    ws = [randn(n, 256, gen=gen, dtype=dtype, scale=0.05) for n in (256, 64, 64)]
    dys = [randn(2, 40, n, gen=gen, dtype=dtype) for n in (256, 64, 64)]
    xd = x.cuda().requires_grad_()
    wd = [w.cuda().requires_grad_() for w in ws]
    ys = shared_input_projections(xd, wd)
    grads = torch.autograd.grad(ys, [xd, *wd], [d.cuda() for d in dys])
    xr = x.double().requires_grad_()
    wr = [w.double().requires_grad_() for w in ws]
    yr = [xr @ w.t() for w in wr]
    er = torch.autograd.grad(yr, [xr, *wr], [d.double() for d in dys])
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    for a, e in zip(list(ys) + list(grads), yr + list(er)):
        assert max_rel(a, e) < tol
        assert cosine(a, e) > 0.999



@pytest.mark.parametrize("m,n,k", [(256, 128, 64), (512, 384, 256), (1024, 1280, 448), (8192, 12288, 4096)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gate_up_swiglu_gemm(m, n, k, dtype):
    """q3_gemm_gate_up_swiglu: G and U bit-equal to the plain GEMM of each weight (same tile and
    k order), Y bit-equal to the SwiGLU kernel on them, and sampled rows against fp64."""
    from qwen3_triton.kernels import _ops
    from qwen3_triton.kernels.linear import gate_up_swiglu_into
    import oracle as O
    print(f"gate_up_swiglu {m}x{n}x{k} {dtype}", flush=True)
    gen = seeded(m + n + k)
    x = randn(m, k, gen=gen, dtype=dtype).cuda()
    wg = randn(n, k, gen=gen, dtype=dtype, scale=0.05).cuda()
    wu = randn(n, k, gen=gen, dtype=dtype, scale=0.05).cuda()
    g, u, y = (torch.empty(m, n, device="cuda", dtype=dtype) for _ in range(3))
    gate_up_swiglu_into(x, wg, wu, g, u, y, m, n, k)
    g2, u2 = torch.empty_like(g), torch.empty_like(u)
    gemm_nt_into(x, k, wg, k, g2, m, n, k)
    gemm_nt_into(x, k, wu, k, u2, m, n, k)
    if m * n >= 256 * 256 * 256:   # the plain GEMM picks the same 256 x 256 tile there
        assert torch.equal(g, g2) and torch.equal(u, u2)
    else:
        assert max_rel(g, g2) <= 8e-3 and max_rel(u, u2) <= 8e-3
    assert torch.equal(y, _ops.swiglu_fwd(g, u))
    rows = torch.arange(0, m, max(1, m // 64))
    xr = x[rows].cpu().double()
    eg, eu = xr @ wg.cpu().double().t(), xr @ wu.cpu().double().t()
    tol = 8e-3 if dtype == torch.bfloat16 else 1e-3
    assert max_rel(g[rows], eg) <= tol and max_rel(u[rows], eu) <= tol
    assert max_rel(y[rows], O.swiglu_reference(eg, eu, dtype=torch.float64)) <= 2 * tol
    # the variant that also stores Y^T: G, U, Y unchanged bit for bit, Y^T exactly Y transposed
    from qwen3_triton.kernels.linear import gate_up_swiglu_t_into
    g3, u3, y3 = (torch.full((m, n), 7.0, device="cuda", dtype=dtype) for _ in range(3))
    yt = torch.full((n, m + 8), 7.0, device="cuda", dtype=dtype)  # row pitch wider than M
    gate_up_swiglu_t_into(x, wg, wu, g3, u3, y3, yt, m, n, k)
    assert torch.equal(g3, g) and torch.equal(u3, u) and torch.equal(y3, y)
    assert torch.equal(yt[:, :m], y.t()) and bool((yt[:, m:] == 7.0).all())
    # Y alone (null G / U: inference): the same Y bit for bit, and the op without autograd gives it too
    y4 = torch.full((m, n), 7.0, device="cuda", dtype=dtype)
    gate_up_swiglu_into(x, wg, wu, None, None, y4, m, n, k)
    assert torch.equal(y4, y)
    with pytest.raises(RuntimeError):   # G and U are stored together or not at all
        gate_up_swiglu_into(x, wg, wu, g3, None, y4, m, n, k)
    from qwen3_triton.kernels.mlp_precision import gate_up_swiglu
    with torch.no_grad():
        assert torch.equal(gate_up_swiglu(x, wg, wu), y)


@pytest.mark.parametrize("m,ns,k", [(256, (256,), 64), (512, (512, 256, 256), 128), (8192, (4096, 1024, 1024), 4096),
                                    (2048, (4096, 1024, 1024), 4096), (384, (128, 256), 64)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_nt_multi(m, ns, k, dtype):
    """One launch over up to 3 weights (the q/k/v projections): every output equals its own q3_gemm_nt
    product bit for bit, and matches fp64 within one rounding."""
    from qwen3_triton.kernels.linear import gemm_nt_multi_into
    print(f"gemm_nt_multi {m}x{ns}x{k} {dtype}", flush=True)
    gen = seeded(m + sum(ns) + k)
    a = randn(m, k, gen=gen, dtype=dtype).cuda()
    ws = [randn(n, k, gen=gen, dtype=dtype).cuda() for n in ns]
    outs = [torch.empty(m, n, device="cuda", dtype=dtype) for n in ns]
    gemm_nt_multi_into(a, ws, outs, m, k)
    for w, o in zip(ws, outs):
        single = torch.empty_like(o)
        gemm_nt_into(a, k, w, k, single, m, w.shape[0], k)
        assert torch.equal(o, single)
        if m <= 512:
            assert max_rel(o, ref(a.cpu(), w.cpu().t())) < 8e-3


@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (512, 768, 256), (8192, 12288, 4096)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("transposed", [True, False])
def test_swiglu_bwd_gemm(m, n, k, dtype, transposed):
    """q3_gemm_swiglu_bwd: dg / du bit-equal to q3_gemm_nt (same 256 x 256 tile where the plain GEMM
    picks it) followed by q3_swiglu_bwd, the transposed copies bit-equal to dg^T / du^T, and sampled
    rows against the fp64 SwiGLU backward of the fp64 product."""
    from qwen3_triton.kernels import _ops
    from qwen3_triton.kernels.linear import swiglu_bwd_gemm_into
    import oracle as O
    print(f"swiglu_bwd_gemm {m}x{n}x{k} {dtype} transposed={transposed}", flush=True)
    gen = seeded(m + 3 * n + k)
    dy = randn(m, k, gen=gen, dtype=dtype).cuda()
    wt = randn(n, k, gen=gen, dtype=dtype, scale=0.05).cuda()
    g = randn(m, n, gen=gen, dtype=dtype).cuda()
    u = randn(m, n, gen=gen, dtype=dtype).cuda()
    dgu = torch.full((m, 2 * n), 7.0, device="cuda", dtype=dtype)
    dgut = torch.full((2 * n, m), 7.0, device="cuda", dtype=dtype) if transposed else None
    swiglu_bwd_gemm_into(dy, wt, g, u, dgu[:, :n], dgu[:, n:], None if dgut is None else dgut[:n],
                         None if dgut is None else dgut[n:], m, n, k)
    dY = torch.empty(m, n, device="cuda", dtype=dtype)
    gemm_nt_into(dy, k, wt, k, dY, m, n, k)
    eg, eu = _ops.swiglu_bwd(g, u, dY)
    if m * n >= 256 * 256 * 256:   # the plain GEMM picks the same 256 x 256 tile there
        assert torch.equal(dgu[:, :n], eg) and torch.equal(dgu[:, n:], eu)
    else:
        assert max_rel(dgu[:, :n], eg) <= 2e-2 and max_rel(dgu[:, n:], eu) <= 2e-2
    if transposed:
        assert torch.equal(dgut[:n], dgu[:, :n].t()) and torch.equal(dgut[n:], dgu[:, n:].t())
    rows = torch.arange(0, m, max(1, m // 64))
    e_dy = dy[rows].cpu().double() @ wt.cpu().double().t()
    rg, ru = O.swiglu_backward_reference(g[rows].cpu().double(), u[rows].cpu().double(), e_dy, dtype=torch.float64)
    tol = 3e-2 if dtype == torch.bfloat16 else 3e-3
    assert max_rel(dgu[rows, :n], rg) <= tol and max_rel(dgu[rows, n:], ru) <= tol


@pytest.mark.parametrize("b,s,h,i", [(2, 256, 256, 768), (1, 512, 512, 1024)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mlp_block_matches_composition(b, s, h, i, dtype):
    """mlp_block (fused SwiGLU backward in the down projection's dX GEMM) gives the outputs and every
    gradient of gate_up_swiglu + linear bit for bit, and matches the fp64 oracle MLP."""
    from qwen3_triton.kernels.mlp_precision import gate_up_swiglu, mlp_block
    import oracle as O
    print(f"mlp_block b{b} s{s} h{h} i{i} {dtype}", flush=True)
    gen = seeded(b * s + h + i)
    x0 = randn(b, s, h, gen=gen, dtype=dtype)
    ws = [randn(i, h, gen=gen, dtype=dtype, scale=0.05), randn(i, h, gen=gen, dtype=dtype, scale=0.05),
          randn(h, i, gen=gen, dtype=dtype, scale=0.05)]
    dout = randn(b, s, h, gen=gen, dtype=dtype)
    res = []
    for fused in (True, False):
        x = x0.cuda().requires_grad_()
        wg, wu, wd = (w.cuda().requires_grad_() for w in ws)
        if fused:
            y = mlp_block(x, wg, wu, wd)
        else:
            from qwen3_triton.kernels.linear import linear
            y = linear(gate_up_swiglu(x, wg, wu), wd)
        y.backward(dout.cuda())
        res.append([y.detach(), x.grad, wg.grad, wu.grad, wd.grad])
    for a, e in zip(*res):
        assert torch.equal(a, e)
    xr = x0.double().requires_grad_()
    wr = [w.double().requires_grad_() for w in ws]
    er = O.swiglu_reference(xr @ wr[0].t(), xr @ wr[1].t(), dtype=torch.float64) @ wr[2].t()
    eg = torch.autograd.grad(er, [xr, *wr], dout.double())
    tol = 2e-2 if dtype == torch.bfloat16 else 3e-3
    assert max_rel(res[0][0], er) <= tol
    for a, e in zip(res[0][1:], eg):
        assert cosine(a, e) >= 0.999


@pytest.mark.parametrize("m,n,k", [(4096, 4096, 256), (8192, 4096, 4096), (2048, 4096, 4096), (2048, 4096, 12288),
                                   (256, 384, 128), (384, 128, 64)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_nt_residual(m, n, k, dtype):
    """q3_gemm_nt_residual: bit-equal to q3_gemm_nt followed by q3_add (in place on the residual too),
    and within one rounding of the fp64 sum.  Shapes with a workspace plan (two K halves) give, through
    q3_gemm_nt_residual_ws, exactly R + (P0 + P1) rounded like the unsplit path, P0 / P1 the fp32
    products of the K halves; without the workspace they stay bit-equal to the GEMM + add."""
    from qwen3_triton import _hip as H
    from qwen3_triton.kernels import _ops
    from qwen3_triton.kernels.linear import gemm_nt_residual_into
    print(f"gemm_nt_residual {m}x{n}x{k} {dtype}", flush=True)
    gen = seeded(m + 5 * n + k)
    a = randn(m, k, gen=gen, dtype=dtype).cuda()
    w = randn(n, k, gen=gen, dtype=dtype, scale=0.05).cuda()
    r = randn(m, n, gen=gen, dtype=dtype).cuda()
    out = torch.empty(m, n, device="cuda", dtype=dtype)
    gemm_nt_residual_into(a, k, w, k, r, out, m, n, k)
    y = torch.empty_like(out)
    gemm_nt_into(a, k, w, k, y, m, n, k)
    e = _ops.add(r, y)
    split = H.query("q3_gemm_nt_residual_workspace_bytes", m, n, k) > 0
    assert split == (m == 2048 and n == 4096 and k >= 8192)
    if split:
        p = [torch.empty(m, n, device="cuda", dtype=torch.float32) for _ in range(2)]
        gemm_nt_into(a, k, w, k, p[0], m, n, k // 2)
        gemm_nt_into(a[:, k // 2:], k, w[:, k // 2:], k, p[1], m, n, k // 2)
        es = ((p[0] + p[1]).to(dtype).float() + r.float()).to(dtype)
        assert torch.equal(out, es)
        plain = torch.empty_like(out)
        H.call("q3_gemm_nt_residual", H.code(dtype), a.data_ptr(), k, w.data_ptr(), k, r.data_ptr(), n,
               plain.data_ptr(), n, m, n, k, H.stream())
        assert torch.equal(plain, e)
        need = H.query("q3_gemm_nt_residual_workspace_bytes", m, n, k)
        short = torch.empty(need, dtype=torch.uint8, device="cuda")
        with pytest.raises(RuntimeError):   # a workspace below the stated size is refused before any launch
            H.call("q3_gemm_nt_residual_ws", H.code(dtype), a.data_ptr(), k, w.data_ptr(), k, r.data_ptr(), n,
                   plain.data_ptr(), n, m, n, k, short.data_ptr(), need - 16, H.stream())
        e = es
    else:
        assert torch.equal(out, e)
    r2 = r.clone()
    gemm_nt_residual_into(a, k, w, k, r2, r2, m, n, k)   # C aliasing R
    assert torch.equal(r2, e)
    # with the next RMSNorm: the same C, and Y = rms_norm(C) (the fused pass sums the squares in its
    # own order: a last-bit difference in 1 / rms may move a few elements by one rounding step)
    from qwen3_triton.kernels.linear import gemm_nt_residual_norm_into
    nw = randn(n, gen=gen, dtype=dtype).cuda()
    c3, y3 = torch.empty_like(out), torch.empty_like(out)
    gemm_nt_residual_norm_into(a, k, w, k, r, c3, nw, 1e-6, y3, m, n, k)
    assert torch.equal(c3, e)
    yr = _ops.rmsnorm_fwd(c3, nw, 1e-6)
    assert (y3 != yr).float().mean().item() < 0.01 and max_rel(y3, yr) <= (8e-3 if dtype == torch.bfloat16 else 1e-3)
    rows = torch.arange(0, m, max(1, m // 64))
    ref64 = r[rows].cpu().double() + a[rows].cpu().double() @ w.cpu().double().t()
    assert max_rel(out[rows], ref64) <= (1.6e-2 if dtype == torch.bfloat16 else 2e-3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gate_up_swiglu_triton_op(dtype):
    """``ops/triton/gate_up_swiglu.py:274-288``: a strided [B, S, K] input (taken as a contiguous copy, as
    the reference takes it) gives the module path's output and gradients bit for bit, and matches the
    fp64 SwiGLU of the fp64 products; the reference's argument errors are raised."""
    import oracle as O
    from ops.triton.gate_up_swiglu import gate_up_swiglu_triton
    from qwen3_triton.kernels.mlp_precision import gate_up_swiglu
    print(f"gate_up_swiglu_triton {dtype}", flush=True)
    gen = seeded(41)
    b, s, k, n = 2, 128, 256, 384
    xs = randn(b, k, s, gen=gen, dtype=dtype).cuda().transpose(1, 2)        # [B, S, K], not contiguous
    wg = randn(n, k, gen=gen, dtype=dtype, scale=0.05).cuda()
    wu = randn(n, k, gen=gen, dtype=dtype, scale=0.05).cuda()
    dy = randn(b, s, n, gen=gen, dtype=dtype).cuda()
    x1 = xs.detach().requires_grad_()
    w1 = [w.detach().requires_grad_() for w in (wg, wu)]
    y1 = gate_up_swiglu_triton(x1, *w1)
    y1.backward(dy)
    x2 = xs.detach().contiguous().requires_grad_()
    w2 = [w.detach().requires_grad_() for w in (wg, wu)]
    y2 = gate_up_swiglu(x2, *w2)
    y2.backward(dy)
    assert torch.equal(y1, y2) and torch.equal(x1.grad, x2.grad)
    assert all(torch.equal(a.grad, c.grad) for a, c in zip(w1, w2))
    xr = xs.detach().cpu().double().reshape(-1, k)
    e = O.swiglu_reference(xr @ wg.cpu().double().t(), xr @ wu.cpu().double().t(), dtype=torch.float64)
    assert max_rel(y1.reshape(-1, n), e) <= (2e-2 if dtype == torch.bfloat16 else 3e-3)
    with pytest.raises(ValueError, match="K dimensions"):
        gate_up_swiglu_triton(xs, wg[:, :128], wu[:, :128])
    with pytest.raises(TypeError, match="same dtype"):
        gate_up_swiglu_triton(xs, wg.float(), wu.float())
    with pytest.raises(ValueError, match="matching weights"):
        gate_up_swiglu_triton(xs, wg, wu[:-1])
