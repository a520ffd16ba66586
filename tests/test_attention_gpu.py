"""Causal GQA flash attention (matrix-core and SIMT paths) vs the CPU oracle and, at the benchmark
shapes, vs torch SDPA in fp32 on the GPU.  Gates: forward max-rel <= 2e-2 (bf16) / 3e-3 (fp16) /
1e-4 (fp32); LSE abs <= 3e-3; gradients cosine >= 0.999 and max-rel <= 4e-2 (bf16)."""
import math

import pytest
import torch
import torch.nn.functional as F

import oracle as O
from _util import cosine, max_rel, randn, seeded

from qwen3_triton.kernels import _ops
from qwen3_triton.kernels.attention import causal_attention
from ops.triton.attention import attention_triton, attention_triton_autograd, attention_triton_qwen_prefill
from ops.triton.attention_backward import attention_backward_triton

pytestmark = pytest.mark.gpu

FWD_TOL = {torch.bfloat16: 2e-2, torch.float16: 3e-3, torch.float32: 1e-4}
GRAD_TOL = {torch.bfloat16: 4e-2, torch.float16: 8e-3, torch.float32: 1e-4}


def make(b, hq, hk, lq, lk, d, dtype, seed):
    gen = seeded(seed)
    q = randn(b, hq, lq, d, gen=gen, dtype=dtype)
    k = randn(b, hk, lk, d, gen=gen, dtype=dtype)
    v = randn(b, hk, lk, d, gen=gen, dtype=dtype)
    do = randn(b, hq, lq, d, gen=gen, dtype=dtype)
    return q, k, v, do


CASES = [(2, 4, 2, 17, 32), (1, 4, 2, 128, 128), (1, 16, 8, 129, 128), (2, 8, 2, 200, 64), (1, 32, 8, 300, 128),
         (1, 2, 2, 1, 128), (2, 4, 1, 65, 32), (1, 4, 2, 33, 48)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("b,hq,hk,s,d", CASES)
def test_attention_fwd_bwd_vs_oracle(b, hq, hk, s, d, dtype):
    print(f"attention {b} {hq} {hk} {s} {d} {dtype}", flush=True)
    q, k, v, do = make(b, hq, hk, s, s, d, dtype, seed=b * 100 + s + d)
    qd, kd, vd = (t.cuda().requires_grad_() for t in (q, k, v))
    o = causal_attention(qd, kd, vd)
    dq, dk, dv = torch.autograd.grad(o, (qd, kd, vd), do.cuda())
    eo = O.scaled_dot_product_attention_reference(q, k, v)
    assert max_rel(o, eo) <= FWD_TOL[dtype]
    _, lse = _ops.attention_fwd(qd.detach(), kd.detach(), vd.detach(), 1 / math.sqrt(d))
    assert (lse.cpu() - O.attention_lse_reference(q, k)).abs().max() <= 3e-3
    e = O.scaled_dot_product_attention_backward_reference(q, k, v, do)
    for a, x, n in zip((dq, dk, dv), e, "qkv"):
        assert cosine(a, x) >= 0.999, f"d{n} cosine"
        assert max_rel(a, x) <= GRAD_TOL[dtype], f"d{n} max-rel {max_rel(a, x)}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("lq,lk", [(1, 1), (1, 300), (7, 129), (64, 1000), (129, 129)])
def test_attention_query_suffix_offset(lq, lk, dtype):
    """Prefill/chunked attention against a longer KV prefix (query i sees keys <= i + lk - lq):
    forward, LSE and the backward (Hq/Hkv = 4, the grouped dK/dV kernel at head_dim 128)."""
    print(f"attention suffix offset lq {lq} lk {lk} {dtype}", flush=True)
    q, k, v, do = make(2, 8, 2, lq, lk, 128, dtype, seed=lq + lk)
    qd, kd, vd, dod = q.cuda(), k.cuda(), v.cuda(), do.cuda()
    o, lse = _ops.attention_fwd(qd, kd, vd, 128 ** -0.5)
    assert max_rel(o, O.scaled_dot_product_attention_reference(q, k, v)) <= FWD_TOL[dtype]
    assert (lse.cpu() - O.attention_lse_reference(q, k)).abs().max() <= 3e-3
    grads = _ops.attention_bwd(qd, kd, vd, o, lse, dod, 128 ** -0.5)
    e = O.scaled_dot_product_attention_backward_reference(q, k, v, do)
    for a, x, n in zip(grads, e, "qkv"):
        assert cosine(a, x) >= 0.999, f"d{n} cosine {cosine(a, x)}"
        assert max_rel(a, x) <= GRAD_TOL[dtype], f"d{n} max-rel {max_rel(a, x)}"


def test_reference_entry_points_agree():
    q, k, v, do = make(1, 4, 2, 128, 128, 128, torch.bfloat16, seed=11)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    o1 = attention_triton(qd, kd, vd)
    o2, lse = attention_triton(qd, kd, vd, return_lse=True)
    o3 = attention_triton_qwen_prefill(qd, kd, vd)
    assert torch.equal(o1, o2) and torch.equal(o1, o3)
    g1 = attention_backward_triton(qd, kd, vd, do.cuda(), lse=lse)
    a = [t.requires_grad_() for t in (qd.clone(), kd.clone(), vd.clone())]
    g2 = torch.autograd.grad(attention_triton_autograd(*a), a, do.cuda())
    for x, y in zip(g1, g2):
        assert torch.equal(x, y)
    g3 = attention_backward_triton(qd, kd, vd, do.cuda(), lse=lse, out=o1)   # saved O: no forward rerun
    for x, y in zip(g3, g2):
        assert torch.equal(x, y)
    from qwen3_triton.kernels.attention_precision import candidate
    assert torch.equal(candidate(qd, kd, vd), o1)
    with pytest.raises(TypeError):
        candidate(qd, kd, vd, lse_fma=1)
    with pytest.raises(NotImplementedError):
        attention_triton(qd, kd, vd, is_causal=False)


def test_attention_invariants_full_shape():
    """V constant -> O constant; row 0 -> V[0] (B4 S2048 Hq32 Hkv8 D128)."""
    gen = seeded(2)
    q = randn(4, 32, 2048, 128, gen=gen, dtype=torch.bfloat16).cuda()
    k = randn(4, 8, 2048, 128, gen=gen, dtype=torch.bfloat16).cuda()
    v = torch.full((4, 8, 2048, 128), 0.75, dtype=torch.bfloat16, device="cuda")
    o, _ = _ops.attention_fwd(q, k, v, 128 ** -0.5)
    assert bool((o == 0.75).all())
    v = randn(4, 8, 2048, 128, gen=gen, dtype=torch.bfloat16).cuda()
    o, _ = _ops.attention_fwd(q, k, v, 128 ** -0.5)
    assert torch.equal(o[:, :, 0], v.repeat_interleave(4, 1)[:, :, 0])


@pytest.mark.parametrize("b,s", [(4, 2048), (1, 8192), (1, 2048)])
def test_attention_benchmark_shapes_vs_sdpa_fp32(b, s):
    """Config #3 shapes against torch SDPA in fp32 on the GPU (a library routine as the checker); B1 S2048
    (the 2048-token prefill) runs the forward's 4-wave workgroups, the other two its 8-wave ones."""
    print(f"attention full {b}x{s}", flush=True)
    gen = seeded(2)
    q = randn(b, 32, s, 128, gen=gen, dtype=torch.bfloat16).cuda()
    k = randn(b, 8, s, 128, gen=gen, dtype=torch.bfloat16).cuda()
    v = randn(b, 8, s, 128, gen=gen, dtype=torch.bfloat16).cuda()
    do = randn(b, 32, s, 128, gen=gen, dtype=torch.bfloat16).cuda()
    qd, kd, vd = (t.clone().requires_grad_() for t in (q, k, v))
    o = causal_attention(qd, kd, vd)
    dq, dk, dv = torch.autograd.grad(o, (qd, kd, vd), do)
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.MATH):
        eo = F.scaled_dot_product_attention(qf, kf, vf, is_causal=True, enable_gqa=True)
    e = torch.autograd.grad(eo, (qf, kf, vf), do.float())
    assert max_rel(o, eo) <= 2e-2
    for a, x in zip((dq, dk, dv), e):
        assert cosine(a, x) >= 0.999
        assert max_rel(a, x) <= 4e-2


def test_attention_strided_layouts_bshd_and_cache():
    """[B,S,H,D] views and a capacity-strided KV cache are read in place (no layout copies)."""
    from qwen3_triton.kernels.attention import causal_attention_bshd
    gen = seeded(21)
    q = randn(2, 40, 8, 128, gen=gen, dtype=torch.bfloat16)
    k = randn(2, 40, 2, 128, gen=gen, dtype=torch.bfloat16)
    v = randn(2, 40, 2, 128, gen=gen, dtype=torch.bfloat16)
    do = randn(2, 40, 8, 128, gen=gen, dtype=torch.bfloat16)
    qd, kd, vd = (t.cuda().requires_grad_() for t in (q, k, v))
    o = causal_attention_bshd(qd, kd, vd)
    grads = torch.autograd.grad(o, (qd, kd, vd), do.cuda())
    qh, kh, vh, dh = (t.transpose(1, 2) for t in (q, k, v, do))
    assert max_rel(o.transpose(1, 2), O.scaled_dot_product_attention_reference(qh, kh, vh)) <= 2e-2
    e = O.scaled_dot_product_attention_backward_reference(qh, kh, vh, dh)
    for a, x in zip(grads, e):
        assert cosine(a.transpose(1, 2), x) >= 0.999
    # cache layout [B,Hkv,C,D] with C > L, queries as the suffix of the key range
    cache_k = torch.zeros(2, 2, 100, 128, dtype=torch.bfloat16)
    cache_v = torch.zeros(2, 2, 100, 128, dtype=torch.bfloat16)
    cache_k[:, :, :40] = kh
    cache_v[:, :, :40] = vh
    ck, cv = cache_k.cuda(), cache_v.cuda()
    oq, _ = _ops.attention_fwd(qh[:, :, 30:].cuda(), ck[:, :, :40], cv[:, :, :40], 128 ** -0.5)
    assert max_rel(oq, O.scaled_dot_product_attention_reference(qh[:, :, 30:], kh, vh)) <= 2e-2


@pytest.mark.parametrize("l", [1, 15, 16, 100, 2048])
@pytest.mark.parametrize("d,layout", [(128, "bhsd"), (64, "bshd"), (32, "bhsd"), (128, "bshd")])
def test_seq_major_layout(l, d, layout):
    """Sequence-major operand copy: [B,H,L,D] -> [B,H,D,Lp] (Lp = L rounded up to 16, zero pad) with the
    4-position groups 1 and 2 of every 16-block swapped; bit-exact, for contiguous and [B,S,H,D] views
    (vector path for D % 64 == 0, element path otherwise)."""
    from qwen3_triton.kernels import _ops
    print(f"seq_major l={l} d={d} {layout}", flush=True)
    if layout == "bhsd":
        x = torch.randn(2, 3, l, d, generator=seeded(l), dtype=torch.float32).to(torch.bfloat16)
        xd = x.cuda()
    else:
        xs = torch.randn(2, l, 3, d, generator=seeded(l), dtype=torch.float32).to(torch.bfloat16)
        x = xs.transpose(1, 2)
        xd = xs.cuda().transpose(1, 2)
    y = _ops.seq_major(xd).cpu()
    lp = -(-l // 16) * 16
    assert y.shape == (2, 3, d, lp)
    ref = torch.zeros(2, 3, d, lp, dtype=torch.bfloat16)
    ref[..., :l] = x.transpose(2, 3)
    p = torch.arange(lp)
    src = p ^ ((((p >> 2) ^ (p >> 3)) & 1) * 12)
    assert torch.equal(y, ref[..., src])

