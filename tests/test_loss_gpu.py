"""Causal CE on materialised logits and the fused LM-head CE vs the CPU oracle.
Gates: loss relative error <= 1e-3; gradients cosine >= 0.999 and max-rel <= 2e-2 (bf16)."""
import pytest
import torch

import oracle as O
from _util import cosine, max_rel, randn, seeded

from qwen3_triton.kernels import _ops
from qwen3_triton.kernels.lm_head_ce import _chunk_logits, lm_head_cross_entropy
from qwen3_triton.kernels.loss import causal_cross_entropy

pytestmark = pytest.mark.gpu


def labels_for(b, s, v, gen, frac_ignore=0.05):
    y = torch.randint(0, v, (b, s), generator=gen)
    y[torch.rand(b, s, generator=gen) < frac_ignore] = -100
    return y


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("b,s,v", [(2, 6, 11), (1, 512, 151936), (3, 17, 4096), (2, 2, 7)])
def test_causal_ce(b, s, v, dtype):
    print(f"ce {b} {s} {v} {dtype}", flush=True)
    gen = seeded(b + s + v)
    z = randn(b, s, v, gen=gen, dtype=dtype, scale=2.0)
    y = labels_for(b, s, v, gen)
    y[0, 1] = -100
    zd = z.cuda().requires_grad_()
    loss = causal_cross_entropy(zd, y.cuda())
    (dz,) = torch.autograd.grad(loss * 1.3, zd)
    e = O.causal_cross_entropy_reference(z, y)
    assert abs(float(loss) - float(e)) <= 1e-3 * abs(float(e))
    eg = O.causal_cross_entropy_backward_reference(z, y, 1.3)
    assert max_rel(dz, eg) <= (2e-2 if dtype == torch.bfloat16 else 3e-3)
    assert cosine(dz, eg) >= 0.999
    assert bool((dz[:, -1] == 0).all())


def test_causal_ce_label_out_of_range_raises():
    z = torch.randn(1, 4, 10, device="cuda")
    with pytest.raises(ValueError):
        causal_cross_entropy(z, torch.tensor([[1, 2, 10, 3]], device="cuda"))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("b,s,h,v,chunk", [(2, 5, 64, 1000, 256), (2, 64, 256, 4096, 1024), (1, 40, 128, 3000, 3000),
                                           (2, 33, 96, 1234, 500)])
def test_lm_head_ce_vs_oracle(b, s, h, v, chunk, dtype):
    print(f"lmhead {b} {s} {h} {v} {chunk} {dtype}", flush=True)
    gen = seeded(v + s)
    x = randn(b, s, h, gen=gen, dtype=dtype)
    w = randn(v, h, gen=gen, dtype=dtype, scale=0.05)
    y = labels_for(b, s, v, gen)
    xd, wd = x.cuda().requires_grad_(), w.cuda().requires_grad_()
    loss = lm_head_cross_entropy(xd, wd, y.cuda(), chunk=chunk)
    dx, dw = torch.autograd.grad(loss, (xd, wd))
    el, ex, ew = O.lm_head_cross_entropy_reference(x, w, y, want_grad=True)
    assert abs(float(loss) - float(el)) <= 1e-3 * abs(float(el))
    for a, e in ((dx, ex), (dw, ew)):
        assert cosine(a, e) >= 0.999
        assert max_rel(a, e) <= (2e-2 if dtype == torch.bfloat16 else 1e-4)


def test_lm_head_ce_config_shape_sampled_rows():
    """Config #4 head: 8192 tokens x 4096 -> 151936.  The full CPU oracle is out of reach, so 24
    sampled rows' losses and dH rows are checked against fp64 on the host; the GPU loss is the mean
    of the per-row losses (checked exactly), and dW rows for sampled vocabulary ids are checked with
    the host-verified per-row lse."""
    gen = seeded(3)
    b, s, h, v = 4, 2048, 4096, 151936
    x = randn(b, s, h, gen=gen, dtype=torch.bfloat16)
    w = randn(v, h, gen=gen, dtype=torch.bfloat16, scale=0.02)
    y = labels_for(b, s, v, gen)
    xd, wd, yd = x.cuda().requires_grad_(), w.cuda().requires_grad_(), y.cuda()
    loss = lm_head_cross_entropy(xd, wd, yd)
    dx, dw = torch.autograd.grad(loss, (xd, wd))
    # per-row pieces from the unfused kernels on the same bf16 logits (the fused path keeps the logits
    # in bf16, the reference's lm_head output dtype, and forms its statistics from them)
    tgt = _ops.ce_shift_labels(yd, -100)
    st = _ops.CEState(b * s, 10, "cuda")
    zbuf = torch.empty(b * s, 16384, device="cuda")
    xf = xd.detach().view(-1, h)
    for c in range(10):
        n = min(16384, v - c * 16384)
        _chunk_logits(xf, wd.detach(), c * 16384, n, zbuf)
        zb = zbuf.to(torch.bfloat16)
        st.stats(c, zb, 16384, n, c * 16384, tgt)
    st.finish(tgt, v, -100)
    assert abs(float(st.loss) - float(loss)) <= 1e-6 * abs(float(loss))
    rows = torch.randperm(b * s, generator=gen)[:24]
    xr = x.view(-1, h)[rows].double()
    z = xr @ w.double().t()
    lse = torch.logsumexp(z, -1)
    tg = tgt.cpu()[rows]
    assert (st.lse.cpu()[rows].double() - lse).abs().max() < 2e-3
    valid = tg != -100
    # the target logit as the bf16 logits hold it (the reference's lm_head output is bf16 as well)
    zt = z.gather(1, tg.clamp_min(0)[:, None])[:, 0].to(torch.bfloat16).double()
    el = torch.where(valid, lse - zt, torch.zeros_like(lse))
    assert (st.loss_rows.cpu()[rows].double() - el).abs().max() < 2e-3
    count = float((tgt != -100).sum())
    p = torch.softmax(z, -1)
    p[valid.nonzero()[:, 0], tg[valid]] -= 1
    p *= valid[:, None].double() / count
    edx = p @ w.double()
    assert cosine(dx.view(-1, h)[rows.cuda()], edx) >= 0.999
    # dW rows for 8 vocabulary ids, using the GPU lse of all rows
    vids = torch.randperm(v, generator=gen)[:8]
    zc = x.view(-1, h).double() @ w[vids].double().t()           # [T, 8]
    tall = tgt.cpu()
    pc = torch.exp(zc - st.lse.cpu().double()[:, None]) - (tall[:, None] == vids[None, :]).double()
    pc *= (tall != -100).double()[:, None] / count
    edw = pc.t() @ x.view(-1, h).double()
    assert cosine(dw[vids.cuda()], edw) >= 0.999


@pytest.mark.parametrize("t,h,n,col0,with_up", [(512, 256, 1000, 3000, True), (300, 128, 4096, 0, False),
                                                (1024, 512, 2304, 8192, True), (8192, 256, 2048, 512, True),
                                                (4096, 128, 4096, 0, False)])
def test_fused_ce_grad_gemm_matches_two_step(t, h, n, col0, with_up):
    """The logits GEMM with the CE-gradient epilogue writes bit-for-bit the dz of the unfused path
    (fp32 logits from the GEMM, then the CE gradient kernel), including ignored and out-of-range rows."""
    print(f"fused ce grad t={t} h={h} n={n} col0={col0}", flush=True)
    gen = seeded(t + n)
    v = col0 + n + 17
    x = randn(t, h, gen=gen, dtype=torch.bfloat16).cuda()
    w = (randn(v, h, gen=gen) * 0.05).to(torch.bfloat16).cuda()
    tgt = torch.randint(0, v, (t,), generator=gen)
    tgt[::7] = -100                      # ignored
    tgt[1::11] = col0 + torch.randint(0, n, (len(tgt[1::11]),), generator=gen)   # targets in this chunk
    tgt[5] = v + 3                       # out of range: treated as ignored here
    tgt = tgt.cuda()
    lse = (randn(t, gen=gen) + 4.0).cuda()
    count = torch.tensor([float((tgt != -100).sum())], device="cuda")
    up = torch.tensor([0.75], device="cuda") if with_up else None
    dz_fused = torch.full((t, n + 8), 7.0, device="cuda", dtype=torch.bfloat16)
    _ops.gemm_ce_grad(x, w, col0, n, tgt, lse, count, up, dz_fused, v, -100)
    z = torch.empty(t, n, device="cuda", dtype=torch.float32)
    _chunk_logits(x, w, col0, n, z)
    dz_ref = torch.empty(t, n, device="cuda", dtype=torch.bfloat16)
    _ops.ce_grad(z, n, n, col0, tgt, lse, count, up, dz_ref, n, v, -100)
    assert torch.equal(dz_fused[:, :n].cpu(), dz_ref.cpu())
    assert torch.all(dz_fused[:, n:].float() == 7.0)          # columns past n untouched
    if _ops.ce_grad_transposed_ok(x, t, n, n + 8, dz_fused, torch.empty(0, t + 8, device="cuda")):
        # the same launch with the transposed copy: dz unchanged, dzt = dz^T, nothing past t written
        dz2 = torch.full((t, n + 8), 7.0, device="cuda", dtype=torch.bfloat16)
        dzt = torch.full((n, t + 8), 5.0, device="cuda", dtype=torch.bfloat16)
        _ops.gemm_ce_grad(x, w, col0, n, tgt, lse, count, up, dz2, v, -100, dzt=dzt)
        assert torch.equal(dz2, dz_fused)
        assert torch.equal(dzt[:, :t], dz_ref.t())
        assert torch.all(dzt[:, t:].float() == 5.0)


@pytest.mark.parametrize("t,h,v,chunk", [(512, 256, 5000, 2048), (300, 128, 4096, 4096), (1024, 512, 9000, 4100),
                                         (256, 64, 8576, 4096)])
def test_fused_ce_stats_gemm_matches_two_step(t, h, v, chunk):
    """The logits GEMM with the statistics epilogue (one partial per 128 logit columns) gives the same
    lse and loss as fp32 logits + the chunk statistics kernel, to fp32 rounding of the merge order."""
    print(f"fused ce stats t={t} h={h} v={v} chunk={chunk}", flush=True)
    gen = seeded(t + v)
    x = randn(t, h, gen=gen, dtype=torch.bfloat16).cuda()
    w = (randn(v, h, gen=gen) * 0.05).to(torch.bfloat16).cuda()
    tgt = torch.randint(0, v, (t,), generator=gen)
    tgt[::9] = -100
    tgt = tgt.cuda()
    nch = -(-v // chunk)
    groups = [-(-min(chunk, v - c * chunk) // 128) for c in range(nch)]
    fused = _ops.CEState(t, sum(groups), x.device)
    part0 = 0
    for c in range(nch):
        fused.gemm_stats(part0, x, w, c * chunk, min(chunk, v - c * chunk), tgt)
        part0 += groups[c]
    loss_f = fused.finish(tgt, v, -100).clone()
    ref = _ops.CEState(t, nch, x.device)
    z = torch.empty(t, chunk, device="cuda", dtype=torch.float32)
    for c in range(nch):
        n = min(chunk, v - c * chunk)
        _chunk_logits(x, w, c * chunk, n, z)
        ref.stats(c, z, chunk, n, c * chunk, tgt)
    loss_r = ref.finish(tgt, v, -100).clone()
    valid = (tgt != -100).cpu()
    assert max_rel(fused.lse.cpu()[valid], ref.lse.cpu()[valid].double()) < 1e-6
    assert abs(float(loss_f) - float(loss_r)) <= 1e-6 * abs(float(loss_r))


@pytest.mark.parametrize("t,h,v,chunk", [(512, 256, 5000, 2048), (1024, 512, 9000, 4096), (256, 64, 8576, 4096)])
def test_fused_ce_stats_store_matches_rounded_two_step(t, h, v, chunk):
    """The statistics GEMM that also stores the logits: the stored chunk is the fp32 GEMM logits rounded
    to bf16 bit for bit (full and ragged tiles), and lse / loss equal the statistics of those rounded
    logits to fp32 rounding of the merge order."""
    print(f"fused ce stats store t={t} h={h} v={v} chunk={chunk}", flush=True)
    gen = seeded(t + v + 1)
    x = randn(t, h, gen=gen, dtype=torch.bfloat16).cuda()
    w = (randn(v, h, gen=gen) * 0.05).to(torch.bfloat16).cuda()
    tgt = torch.randint(0, v, (t,), generator=gen)
    tgt[::9] = -100
    tgt = tgt.cuda()
    nch = -(-v // chunk)
    groups = [-(-min(chunk, v - c * chunk) // 128) for c in range(nch)]
    fused = _ops.CEState(t, sum(groups), x.device)
    vp = -(-v // 64) * 64
    zs = torch.full((t, vp), 3.0, device="cuda", dtype=torch.bfloat16)
    part0 = 0
    for c in range(nch):
        fused.gemm_stats_store(part0, x, w, c * chunk, min(chunk, v - c * chunk), tgt, zs[:, c * chunk:])
        part0 += groups[c]
    loss_f = fused.finish(tgt, v, -100).clone()
    ref = _ops.CEState(t, nch, x.device)
    z = torch.empty(t, chunk, device="cuda", dtype=torch.float32)
    for c in range(nch):
        n = min(chunk, v - c * chunk)
        _chunk_logits(x, w, c * chunk, n, z)
        zb = z.to(torch.bfloat16)
        assert torch.equal(zs[:, c * chunk:c * chunk + n], zb[:, :n])
        ref.stats(c, zb, chunk, n, c * chunk, tgt)
    assert torch.all(zs[:, v:].float() == 3.0)                  # nothing past the vocabulary written
    loss_r = ref.finish(tgt, v, -100).clone()
    valid = (tgt != -100).cpu()
    assert max_rel(fused.lse.cpu()[valid], ref.lse.cpu()[valid].double()) < 1e-6
    assert abs(float(loss_f) - float(loss_r)) <= 1e-6 * abs(float(loss_r))


@pytest.mark.parametrize("t,n,col0,inplace", [(512, 1000, 3000, False), (8192, 16384, 0, True),
                                              (64, 4480, 147456, True), (24, 136, 8, False)])
def test_ce_grad_transposed_matches_chunk_grad(t, n, col0, inplace):
    """dz from stored bf16 logits with its transpose (q3_ce_chunk_grad_t) equals q3_ce_chunk_grad on the
    same logits bit for bit, in place or not, with ignored and in-chunk targets; dzt = dz^T."""
    print(f"ce grad t t={t} n={n} col0={col0} inplace={inplace}", flush=True)
    gen = seeded(t + n + col0)
    v = col0 + n + 9
    ld = n + 24
    z = (randn(t, ld, gen=gen) * 3).to(torch.bfloat16).cuda()
    tgt = torch.randint(0, v, (t,), generator=gen)
    tgt[::7] = -100
    tgt[1::5] = col0 + torch.randint(0, n, (len(tgt[1::5]),), generator=gen)
    tgt = tgt.cuda()
    lse = (randn(t, gen=gen) + 6.0).cuda()
    count = torch.tensor([float((tgt != -100).sum())], device="cuda")
    up = torch.tensor([1.25], device="cuda")
    ref = torch.empty(t, n, device="cuda", dtype=torch.bfloat16)
    _ops.ce_grad(z, ld, n, col0, tgt, lse, count, up, ref, n, v, -100)
    dzt = torch.full((n, t + 8), 5.0, device="cuda", dtype=torch.bfloat16)
    if inplace:
        zc = z.clone()
        _ops.ce_grad_t(zc, n, col0, tgt, lse, count, up, zc, dzt, v, -100)
        dz = zc
        assert torch.equal(zc[:, n:], z[:, n:])                    # columns past n untouched
    else:
        dz = torch.full((t, ld), 7.0, device="cuda", dtype=torch.bfloat16)
        _ops.ce_grad_t(z, n, col0, tgt, lse, count, up, dz, dzt, v, -100)
        assert torch.all(dz[:, n:].float() == 7.0)
    assert torch.equal(dz[:, :n], ref)
    assert torch.equal(dzt[:, :t], ref.t())
    assert torch.all(dzt[:, t:].float() == 5.0)


def test_lm_head_ce_second_backward_recomputes():
    """The stored bf16 logits are consumed (turned into dz in place) by the first backward; a second
    backward through a retained graph recomputes the logits instead, and both give the same gradients
    to the bf16 gate (their logits differ by one bf16 rounding)."""
    gen = seeded(77)
    x = randn(2, 256, 256, gen=gen, dtype=torch.bfloat16).cuda().requires_grad_()
    w = randn(4096, 256, gen=gen, dtype=torch.bfloat16, scale=0.05).cuda().requires_grad_()
    y = labels_for(2, 256, 4096, gen).cuda()
    loss = lm_head_cross_entropy(x, w, y, chunk=1024)
    g1 = torch.autograd.grad(loss, (x, w), retain_graph=True)
    g2 = torch.autograd.grad(loss, (x, w))
    for a, b in zip(g1, g2):
        assert cosine(a, b) >= 0.9999
        assert max_rel(a, b) <= 2e-2
