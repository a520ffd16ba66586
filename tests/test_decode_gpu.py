"""Decode kernels: small-M GEMV, KV append, split-KV decode attention, greedy select."""
import pytest
import torch

import oracle as O
from _util import max_rel, randn, seeded

from qwen3_triton.inference import kernels as K

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m", [1, 2, 5, 8, 16])
@pytest.mark.parametrize("n,k", [(4096, 4096), (1024, 4096), (4096, 12288), (151936, 4096), (37, 64), (5000, 520)])
def test_gemv(m, n, k):
    print(f"gemv m={m} n={n} k={k}", flush=True)
    gen = seeded(m + n + k)
    x = randn(m, k, gen=gen, dtype=torch.bfloat16)
    w = randn(n, k, gen=gen, dtype=torch.bfloat16, scale=0.02)
    y = K.linear(x.cuda(), w.cuda())
    e = x.double() @ w.double().t()
    assert max_rel(y, e) <= 8e-3
    y2 = K.linear(x.cuda(), w.cuda())
    assert torch.equal(y, y2)  # deterministic


@pytest.mark.parametrize("m", [1, 5, 16])
@pytest.mark.parametrize("k", [4096, 688, 256, 12288])
@pytest.mark.parametrize("norm", [False, True])
def test_decode_linear_modes(m, k, norm):
    """Fused decode projection against the unfused fp64 math: xn = bf16(rmsnorm(x)) (the kernel
    rounds x * norm_w instead and applies the row scale to the fp32 dot product: the same math up to
    one bf16 rounding); mode 0 three segments; mode 1 res + bf16(y); mode 2 silu(bf16 g) bf16(u)."""
    print(f"decode_linear m={m} k={k} norm={norm}", flush=True)
    gen = seeded(m * 7 + k + int(norm))
    dt = torch.bfloat16
    x = randn(m, k, gen=gen, dtype=dt)
    nw = (1.0 + 0.1 * randn(k, gen=gen)).to(dt)
    ws = [randn(n, k, gen=gen, dtype=dt, scale=0.02) for n in (1000, 200, 200)]
    res = randn(m, 1000, gen=gen, dtype=dt)
    xn = O.rms_norm_reference(x, nw, 1e-6, dtype=torch.float64).to(dt) if norm else x
    kw = dict(norm_weight=nw.cuda() if norm else None, eps=1e-6)
    ys = K.decode_linear(x.cuda(), [w.cuda() for w in ws], **kw)
    for y, w in zip(ys, ws):
        assert max_rel(y, xn.double() @ w.double().t()) <= 1e-2
    y1 = K.decode_linear(x.cuda(), [ws[0].cuda()], mode=1, res=res.cuda(), **kw)
    e1 = res.double() + (xn.double() @ ws[0].double().t()).to(dt).double()
    assert max_rel(y1, e1) <= 1e-2
    g, u = ws[1], ws[2]
    y2 = K.decode_linear(x.cuda(), [g.cuda(), u.cuda()], mode=2, **kw)
    eg = (xn.double() @ g.double().t()).to(dt)
    eu = (xn.double() @ u.double().t()).to(dt)
    e2 = O.swiglu_reference(eg, eu, dtype=torch.float64)
    assert max_rel(y2, e2) <= 2e-2
    assert torch.equal(y2, K.decode_linear(x.cuda(), [g.cuda(), u.cuda()], mode=2, **kw))  # deterministic


@pytest.mark.parametrize("m", [1, 5, 8, 9])
@pytest.mark.parametrize("k", [4096, 2048, 1024])
@pytest.mark.parametrize("norm", [False, True])
def test_decode_linear_eight_row_units(m, k, norm):
    """Projections with 256 < 16-row tiles <= 512 (the Q/K/V launch) run on 8-row units for at most 8
    token rows: ragged segment ends, every row of every segment checked against fp64 math."""
    print(f"decode_linear 8-row units m={m} k={k} norm={norm}", flush=True)
    gen = seeded(m * 11 + k + int(norm))
    dt = torch.bfloat16
    x = randn(m, k, gen=gen, dtype=dt)
    nw = (1.0 + 0.1 * randn(k, gen=gen)).to(dt)
    ws = [randn(n, k, gen=gen, dtype=dt, scale=0.02) for n in (4096, 1024, 1028)]
    xn = O.rms_norm_reference(x, nw, 1e-6, dtype=torch.float64).to(dt) if norm else x
    ys = K.decode_linear(x.cuda(), [w.cuda() for w in ws], norm_weight=nw.cuda() if norm else None, eps=1e-6)
    for y, w in zip(ys, ws):
        e = xn.double() @ w.double().t()
        assert y.shape == e.shape
        assert max_rel(y, e) <= 1e-2
        # row-wise too: a wrong unit or k-half mapping would corrupt whole rows of a segment
        err = (y.double().cpu() - e).abs().amax(dim=0) / e.abs().amax()
        assert float(err.max()) <= 2e-2


def test_kv_append():
    gen = seeded(1)
    k = randn(2, 5, 3, 128, gen=gen, dtype=torch.bfloat16)
    v = randn(2, 5, 3, 128, gen=gen, dtype=torch.bfloat16)
    ck = torch.zeros(2, 3, 20, 128, dtype=torch.bfloat16, device="cuda")
    cv = torch.zeros_like(ck)
    K.append(k.cuda(), v.cuda(), ck, cv, 7)
    assert torch.equal(ck[:, :, 7:12].cpu(), k.transpose(1, 2))
    assert torch.equal(cv[:, :, 7:12].cpu(), v.transpose(1, 2))
    assert bool((ck[:, :, :7] == 0).all()) and bool((ck[:, :, 12:] == 0).all())


@pytest.mark.parametrize("b,hq,hk,t", [(1, 32, 8, 1), (1, 32, 8, 2048), (8, 32, 8, 1100), (2, 4, 2, 129),
                                       (1, 32, 8, 2304), (1, 8, 8, 300), (2, 24, 8, 70), (1, 16, 2, 500),
                                       (3, 32, 8, 64), (1, 32, 8, 65)])
def test_decode_attention(b, hq, hk, t):
    gen = seeded(t)
    cap = t + 5
    q = randn(b, 1, hq, 128, gen=gen, dtype=torch.bfloat16)
    kk = randn(b, hk, cap, 128, gen=gen, dtype=torch.bfloat16)
    vv = randn(b, hk, cap, 128, gen=gen, dtype=torch.bfloat16)
    out = K.attention(q.cuda(), kk.cuda(), vv.cuda(), t - 1)
    e = O.scaled_dot_product_attention_reference(q.transpose(1, 2), kk[:, :, :t], vv[:, :, :t])
    assert max_rel(out.transpose(1, 2), e) <= 2e-2


def test_decode_attention_lengths():
    """Back-to-back calls of several lengths, device length (whole-capacity launch) against host
    length."""
    gen = seeded(77)
    b, hq, hk, cap = 2, 32, 8, 700
    kk = randn(b, hk, cap, 128, gen=gen, dtype=torch.bfloat16).cuda()
    vv = randn(b, hk, cap, 128, gen=gen, dtype=torch.bfloat16).cuda()
    for t in (650, 1, 129, 700):
        q = randn(b, 1, hq, 128, gen=gen, dtype=torch.bfloat16)
        e = O.scaled_dot_product_attention_reference(q.transpose(1, 2), kk[:, :, :t].cpu(), vv[:, :, :t].cpu())
        out = K.attention(q.cuda(), kk, vv, t - 1)
        assert max_rel(out.transpose(1, 2), e) <= 2e-2
        dev = torch.tensor([t - 1], dtype=torch.int64, device="cuda")
        out2 = K.attention(q.cuda(), kk, vv, 0, start_dev=dev)
        assert max_rel(out2.transpose(1, 2), e) <= 2e-2


@pytest.mark.parametrize("b,hq,hk,t,dev", [(1, 32, 8, 2048, False), (1, 32, 8, 2048, True), (8, 32, 8, 1100, True),
                                           (2, 4, 2, 64, False), (2, 16, 2, 65, True), (1, 8, 8, 1, False)])
def test_decode_step_attention_matches_unfused(b, hq, hk, t, dev):
    """QK-norm + RoPE + cache append + attention in one kernel pair: bit-identical output and caches
    to norm_rope, append and decode attention run separately."""
    print(f"decode_step_attention b={b} hq={hq} hk={hk} t={t} dev={dev}", flush=True)
    gen = seeded(t + hq)
    cap = t + 7
    dt = torch.bfloat16
    q = randn(b, 1, hq, 128, gen=gen, dtype=dt).cuda()
    k = randn(b, 1, hk, 128, gen=gen, dtype=dt).cuda()
    v = randn(b, 1, hk, 128, gen=gen, dtype=dt).cuda()
    qw = (1 + 0.1 * randn(128, gen=gen)).to(dt).cuda()
    kw = (1 + 0.1 * randn(128, gen=gen)).to(dt).cuda()
    ck0 = randn(b, hk, cap, 128, gen=gen, dtype=dt).cuda()
    cv0 = randn(b, hk, cap, 128, gen=gen, dtype=dt).cuda()
    from qwen3_triton.kernels import _ops
    inv = O.rope_inv_freq(1e6, 128)
    cos, sin = _ops.rope_tables(torch.full((b, 1), t - 1, dtype=torch.int64, device="cuda"), inv.cuda(), dt)
    start_dev = torch.tensor([t - 1], dtype=torch.int64, device="cuda") if dev else None
    ck1, cv1 = ck0.clone(), cv0.clone()
    qn = K.norm_rope(q, qw, cos, sin, 1e-6)
    kn = K.norm_rope(k, kw, cos, sin, 1e-6)
    K.append(kn, v, ck1, cv1, t - 1)
    e = K.attention(qn, ck1, cv1, t - 1)
    ck2, cv2 = ck0.clone(), cv0.clone()
    y = K.decode_step_attention(q, k, v, qw, kw, 1e-6, cos, sin, ck2, cv2, 0 if dev else t - 1, start_dev)
    assert torch.equal(ck2, ck1) and torch.equal(cv2, cv1)
    assert torch.equal(y, e)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_greedy_select_ties_pad_eos(dtype):
    v = 151936
    logits = torch.randn(4, v).to(dtype)
    logits[0, 5] = logits[0, 77] = logits[0, 150000] = 100.0   # ties -> lowest index
    logits[1, v - 1] = 50.0
    logits[2, 3] = 60.0
    lg = logits.cuda()
    ids = torch.zeros(4, 10, dtype=torch.int64, device="cuda")
    nxt = torch.empty(4, 1, dtype=torch.int64, device="cuda")
    done = torch.tensor([False, False, True, False], device="cuda")
    K.select(lg, ids, nxt, done, 6, (v - 1,), 9)
    exp = O.argmax_lowest_reference(logits.float())
    assert nxt[:, 0].tolist() == [5, v - 1, 9, int(exp[3])]
    assert ids[:, 6].tolist() == nxt[:, 0].tolist()
    assert done.tolist() == [False, True, True, False]


@pytest.mark.parametrize("b,s,start,cap", [(1, 2048, 0, 2304), (8, 64, 100, 200), (2, 7, 5, 12)])
def test_norm_rope_qk_cache_matches_separate_launches(b, s, start, cap):
    """The prefill launch (Q/K-norm + RoPE of q and k, k and v into the cache) is bit-identical to the
    two QK-norm + RoPE launches followed by the cache append, and leaves other cache positions alone."""
    from qwen3_triton.kernels import _ops
    from qwen3_triton.inference import kernels
    print(f"norm_rope_qk_cache B{b} S{s} start {start} cap {cap}", flush=True)
    gen = seeded(b * 1000 + s)
    r = lambda *sh: torch.randn(*sh, generator=gen).to(torch.bfloat16).cuda()  # noqa: E731
    q, k, v = r(b, s, 32, 128), r(b, s, 8, 128), r(b, s, 8, 128)
    qw, kw = r(128) * 0.1 + 1, r(128) * 0.1 + 1
    pos = torch.arange(start, start + s)[None].expand(b, s)
    cos, sin = O.rotary_tables_reference(pos, O.rope_inv_freq(1e6, 128), dtype=torch.bfloat16)
    cos, sin = cos.cuda(), sin.cuda()
    ck0, cv0 = r(b, 8, cap, 128), r(b, 8, cap, 128)
    ck1, cv1 = ck0.clone(), cv0.clone()
    yq = _ops.norm_rope_qk_cache_fwd(q, k, v, qw, kw, cos, sin, ck1, cv1, start, 1e-6)
    eq = _ops.norm_rope_fwd(q, qw, cos, sin, 1e-6)
    ek = _ops.norm_rope_fwd(k, kw, cos, sin, 1e-6)
    kernels.append(ek, v, ck0, cv0, start)
    torch.cuda.synchronize()
    assert torch.equal(yq, eq)
    assert torch.equal(ck1, ck0) and torch.equal(cv1, cv0)
