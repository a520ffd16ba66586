"""Pins the CPU oracle (oracle/reference.py) before anything is compared against it.

Each oracle function is checked against something independent of its own formula: a known
answer from the reference's tests, a closed form, an invariant, autograd of the forward, or a
third-party library routine (torch.nn.functional, HF transformers' Qwen3 built from a local
config).  A plausible slip (dropped term, wrong sign, transposed operand, off-by-one shift) fails
at least one of these.
"""
import math

import pytest
import torch
import torch.nn.functional as F

import oracle as O

D64 = torch.float64


def g(seed):
    return torch.Generator().manual_seed(seed)


# ------------------------------------------------------------------ RMSNorm
def test_rmsnorm_constant_row_closed_form():
    # x = c everywhere -> y = w * c / sqrt(c^2 + eps)
    for c in (3.0, -0.5):
        x = torch.full((2, 16), c, dtype=D64)
        w = torch.linspace(0.5, 2.0, 16, dtype=D64)
        y = O.rms_norm_reference(x, w, 1e-6, dtype=D64)
        torch.testing.assert_close(y, (w * c / math.sqrt(c * c + 1e-6)).expand(2, 16))


def test_rmsnorm_unit_rms_invariant():
    x = torch.randn(5, 64, generator=g(0), dtype=D64) * 7
    y = O.rms_norm_reference(x, torch.ones(64, dtype=D64), 0.0, dtype=D64)
    torch.testing.assert_close(y.square().mean(-1), torch.ones(5, dtype=D64))


def test_rmsnorm_backward_matches_autograd():
    x = torch.randn(3, 7, 32, generator=g(1), dtype=D64, requires_grad=True)
    w = (1 + 0.1 * torch.randn(32, generator=g(2), dtype=D64)).requires_grad_()
    dy = torch.randn(3, 7, 32, generator=g(3), dtype=D64)
    y = O.rms_norm_reference(x, w, 1e-6, dtype=D64)
    ex, ew = torch.autograd.grad(y, (x, w), dy)
    dx, dw = O.rms_norm_backward_reference(x.detach(), w.detach(), dy, 1e-6, dtype=D64)
    torch.testing.assert_close(dx, ex)
    torch.testing.assert_close(dw, ew)


# ------------------------------------------------------------------ RoPE
def test_rotate_half_known_answer():
    # tests/test_rope.py:12-15 of the reference
    x = torch.arange(8).float()
    torch.testing.assert_close(O.rotate_half_reference(x), torch.tensor([-4., -5., -6., -7., 0., 1., 2., 3.]))
    torch.testing.assert_close(O.inverse_rotate_half_reference(O.rotate_half_reference(x)), x)


def test_rope_tables_match_hf_and_position_zero_is_identity():
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding
    cfg = Qwen3Config(hidden_size=64, num_attention_heads=4, num_key_value_heads=2, head_dim=16,
                      max_position_embeddings=4096, rope_theta=1_000_000.0)
    pos = torch.tensor([[0, 1, 2, 7, 2047], [3, 4, 5, 6, 9]])
    hc, hs = Qwen3RotaryEmbedding(cfg)(torch.zeros(2, 5, 64), pos)
    c, s = O.rotary_tables_reference(pos, O.rope_inv_freq(1e6, 16))
    torch.testing.assert_close(c, hc, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(s, hs, rtol=1e-5, atol=1e-5)
    q = torch.randn(2, 3, 5, 16, generator=g(4))
    rq, _ = O.apply_rope_reference(q, q, c, s)
    torch.testing.assert_close(rq[0, :, 0], q[0, :, 0])          # position 0 (batch 0): identity
    torch.testing.assert_close(rq.norm(dim=-1), q.norm(dim=-1))   # rotation preserves norms


def test_rope_matches_hf_apply():
    from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb
    q = torch.randn(2, 4, 5, 16, generator=g(5))
    k = torch.randn(2, 2, 5, 16, generator=g(6))
    c, s = O.rotary_tables_reference(torch.arange(5)[None].expand(2, 5), O.rope_inv_freq(1e6, 16))
    eq, ek = apply_rotary_pos_emb(q, k, c, s)
    aq, ak = O.apply_rope_reference(q, k, c, s)
    torch.testing.assert_close(aq, eq)
    torch.testing.assert_close(ak, ek)


def test_rope_backward_is_transpose_for_general_tables():
    # independent random cos/sin (not real angles) catch a backward indexing bug
    q = torch.randn(2, 3, 4, 8, generator=g(7), dtype=D64, requires_grad=True)
    c = torch.randn(2, 4, 8, generator=g(8), dtype=D64)
    s = torch.randn(2, 4, 8, generator=g(9), dtype=D64)
    gy = torch.randn(2, 3, 4, 8, generator=g(10), dtype=D64)
    y, _ = O.apply_rope_reference(q, q, c, s, dtype=D64)
    (e,) = torch.autograd.grad(y, q, gy)
    a, _ = O.apply_rope_backward_reference(gy, gy, c, s, dtype=D64)
    torch.testing.assert_close(a, e)


def test_fused_qk_norm_rope_backward_matches_autograd():
    q = torch.randn(2, 5, 4, 16, generator=g(11), dtype=D64, requires_grad=True)
    k = torch.randn(2, 5, 2, 16, generator=g(12), dtype=D64, requires_grad=True)
    qw = (1 + 0.1 * torch.randn(16, generator=g(13), dtype=D64)).requires_grad_()
    kw = (1 + 0.1 * torch.randn(16, generator=g(14), dtype=D64)).requires_grad_()
    c = torch.randn(2, 5, 16, generator=g(15), dtype=D64)
    s = torch.randn(2, 5, 16, generator=g(16), dtype=D64)
    gq = torch.randn(2, 5, 4, 16, generator=g(17), dtype=D64)
    gk = torch.randn(2, 5, 2, 16, generator=g(18), dtype=D64)
    yq, yk = O.fused_qk_norm_rope_reference(q, k, qw, kw, c, s, 1e-6, dtype=D64)
    e = torch.autograd.grad((yq, yk), (q, k, qw, kw), (gq, gk))
    a = O.fused_qk_norm_rope_backward_reference(q.detach(), k.detach(), qw.detach(), kw.detach(), c, s, gq, gk,
                                                1e-6, dtype=D64)
    for x, y in zip(a, e):
        torch.testing.assert_close(x, y)


# ------------------------------------------------------------------ SwiGLU
def test_swiglu_matches_functional_silu_and_autograd():
    gt = torch.randn(4, 33, generator=g(19), dtype=D64, requires_grad=True)
    ut = torch.randn(4, 33, generator=g(20), dtype=D64, requires_grad=True)
    y = O.swiglu_reference(gt, ut, dtype=D64)
    torch.testing.assert_close(y, F.silu(gt) * ut)
    dy = torch.randn(4, 33, generator=g(21), dtype=D64)
    e = torch.autograd.grad(F.silu(gt) * ut, (gt, ut), dy)
    a = O.swiglu_backward_reference(gt.detach(), ut.detach(), dy, dtype=D64)
    torch.testing.assert_close(a[0], e[0])
    torch.testing.assert_close(a[1], e[1])


# ------------------------------------------------------------------ attention
@pytest.mark.parametrize("lq,lk", [(17, 17), (5, 12), (1, 9)])
def test_attention_matches_sdpa_and_lse(lq, lk):
    q = torch.randn(2, 4, lq, 16, generator=g(22), dtype=D64)
    k = torch.randn(2, 2, lk, 16, generator=g(23), dtype=D64)
    v = torch.randn(2, 2, lk, 16, generator=g(24), dtype=D64)
    # SDPA's is_causal uses the top-left convention; build the suffix mask explicitly.
    mask = torch.arange(lk)[None, :] <= (torch.arange(lq) + lk - lq)[:, None]
    e = F.scaled_dot_product_attention(q, k.repeat_interleave(2, 1), v.repeat_interleave(2, 1), attn_mask=mask)
    torch.testing.assert_close(O.scaled_dot_product_attention_reference(q, k, v, dtype=D64), e)
    sc = q @ k.repeat_interleave(2, 1).transpose(-1, -2) / 4.0
    lse = torch.logsumexp(sc.masked_fill(~mask, float("-inf")), -1)
    torch.testing.assert_close(O.attention_lse_reference(q, k, dtype=D64), lse)


def test_attention_invariants():
    q = torch.randn(1, 2, 6, 8, generator=g(25), dtype=D64)
    k = torch.randn(1, 1, 6, 8, generator=g(26), dtype=D64)
    v = torch.randn(1, 1, 6, 8, generator=g(27), dtype=D64)
    o = O.scaled_dot_product_attention_reference(q, k, v, dtype=D64)
    torch.testing.assert_close(o[:, :, 0], v[:, :, 0].expand(1, 2, 8))  # causal row 0 sees only key 0
    vc = torch.full_like(v, 2.5)
    torch.testing.assert_close(O.scaled_dot_product_attention_reference(q, k, vc, dtype=D64),
                               torch.full_like(o, 2.5))


def test_attention_backward_matches_autograd():
    q = torch.randn(2, 4, 9, 8, generator=g(28), dtype=D64, requires_grad=True)
    k = torch.randn(2, 2, 9, 8, generator=g(29), dtype=D64, requires_grad=True)
    v = torch.randn(2, 2, 9, 8, generator=g(30), dtype=D64, requires_grad=True)
    do = torch.randn(2, 4, 9, 8, generator=g(31), dtype=D64)
    o = O.scaled_dot_product_attention_reference(q, k, v, dtype=D64)
    e = torch.autograd.grad(o, (q, k, v), do)
    a = O.scaled_dot_product_attention_backward_reference(q.detach(), k.detach(), v.detach(), do, dtype=D64)
    for x, y in zip(a, e):
        torch.testing.assert_close(x, y)


# ------------------------------------------------------------------ loss
def test_causal_ce_matches_functional_and_uniform_case():
    z = torch.randn(2, 6, 11, generator=g(32), dtype=D64)
    y = torch.randint(0, 11, (2, 6), generator=g(33))
    y[0, 3] = -100
    e = F.cross_entropy(z[:, :-1].reshape(-1, 11), y[:, 1:].reshape(-1), ignore_index=-100)
    torch.testing.assert_close(O.causal_cross_entropy_reference(z, y, dtype=D64), e)
    zu = torch.zeros(1, 4, 50, dtype=D64)
    torch.testing.assert_close(O.causal_cross_entropy_reference(zu, torch.zeros(1, 4, dtype=torch.long),
                                                                dtype=D64), torch.tensor(math.log(50), dtype=D64))


def test_causal_ce_backward_matches_autograd_and_rows_sum_to_zero():
    z = torch.randn(2, 6, 11, generator=g(34), dtype=D64, requires_grad=True)
    y = torch.randint(0, 11, (2, 6), generator=g(35))
    y[1, 2] = -100
    loss = O.causal_cross_entropy_reference(z, y, dtype=D64)
    (e,) = torch.autograd.grad(loss * 1.7, z)
    a = O.causal_cross_entropy_backward_reference(z.detach(), y, 1.7, dtype=D64)
    torch.testing.assert_close(a, e)
    torch.testing.assert_close(a.sum(-1), torch.zeros(2, 6, dtype=D64))


def test_lm_head_ce_matches_materialised_logits_and_grads():
    h = torch.randn(2, 5, 12, generator=g(36), dtype=D64, requires_grad=True)
    w = (0.3 * torch.randn(37, 12, generator=g(37), dtype=D64)).requires_grad_()
    y = torch.randint(0, 37, (2, 5), generator=g(38))
    y[0, 4] = -100
    loss = O.causal_cross_entropy_reference(h @ w.T, y, dtype=D64)
    eh, ew = torch.autograd.grad(loss, (h, w))
    a, ah, aw = O.lm_head_cross_entropy_reference(h.detach(), w.detach(), y, dtype=D64, chunk=8, want_grad=True)
    torch.testing.assert_close(a, loss.detach())
    torch.testing.assert_close(ah, eh)
    torch.testing.assert_close(aw, ew)


def test_embedding_backward_brute_force():
    ids = torch.tensor([[3, 1, 3], [0, 3, 1]])
    gr = torch.randn(2, 3, 5, generator=g(39), dtype=D64)
    out = O.embedding_backward_reference(ids, gr, 6, dtype=D64)
    exp = torch.zeros(6, 5, dtype=D64)
    for b in range(2):
        for s in range(3):
            exp[ids[b, s]] += gr[b, s]
    torch.testing.assert_close(out, exp)


def test_argmax_lowest_index_on_ties():
    x = torch.tensor([[1., 5., 5., 2.], [7., 0., 7., 7.]])
    assert O.argmax_lowest_reference(x).tolist() == [1, 0]


# ------------------------------------------------------------------ model vs HF transformers
def _hf_model(cfg, params):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    hc = Qwen3Config(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
                     intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_hidden_layers,
                     num_attention_heads=cfg.num_attention_heads, num_key_value_heads=cfg.num_key_value_heads,
                     head_dim=cfg.head_dim, rope_theta=cfg.rope_theta, rms_norm_eps=cfg.rms_norm_eps,
                     tie_word_embeddings=cfg.tie_word_embeddings, max_position_embeddings=512,
                     attn_implementation="eager")
    m = Qwen3ForCausalLM(hc).double().eval()
    m.load_state_dict({k: v.double() for k, v in params.items()}, strict=True)
    return m


def test_tiny_model_forward_loss_matches_hf_qwen3():
    cfg = O.OracleConfig(vocab_size=97, hidden_size=32, intermediate_size=40, num_hidden_layers=2,
                         num_attention_heads=4, num_key_value_heads=2, head_dim=8)
    p = O.init_params(cfg, seed=0, std=0.2)
    ids = torch.randint(0, 97, (2, 9), generator=g(40))
    logits, loss = O.model_forward_reference(ids, p, cfg, labels=ids, dtype=D64)
    hf = _hf_model(cfg, p)
    with torch.no_grad():
        out = hf(input_ids=ids, labels=ids)
    # HF's RMSNorm upcasts to fp32 internally even for an fp64 model: agreement is ~1e-7 relative.
    torch.testing.assert_close(logits, out.logits, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(loss, out.loss.double(), rtol=1e-6, atol=1e-6)


def test_greedy_loop_matches_hf_generate():
    cfg = O.OracleConfig(vocab_size=61, hidden_size=32, intermediate_size=40, num_hidden_layers=2,
                         num_attention_heads=4, num_key_value_heads=2, head_dim=8)
    p = O.init_params(cfg, seed=1, std=0.3)
    ids = torch.randint(0, 61, (2, 5), generator=g(41))
    toks, margins = O.greedy_generate_reference(ids, p, cfg, 6, dtype=D64)
    hf = _hf_model(cfg, p)
    with torch.no_grad():
        e = hf.generate(ids, max_new_tokens=6, do_sample=False, eos_token_id=None, pad_token_id=0)
    assert torch.equal(toks, e)
    assert margins.shape == (2, 6) and bool((margins >= 0).all())


def test_cached_decode_matches_full_recomputation():
    """The KV-cached oracle decode (prefill, then one token per step against the cache) equals the
    full-recomputation greedy loop token for token, and every step's logits equal the last row of
    a no-cache forward over the whole prefix (fp64); teacher forcing feeds the given tokens."""
    cfg = O.OracleConfig(vocab_size=61, hidden_size=32, intermediate_size=40, num_hidden_layers=2,
                         num_attention_heads=4, num_key_value_heads=2, head_dim=8)
    p = {k: v.double() for k, v in O.init_params(cfg, seed=3, std=0.3).items()}
    ids = torch.randint(0, 61, (3, 7), generator=g(43))
    full, _ = O.greedy_generate_reference(ids, p, cfg, 5, dtype=D64)
    toks, logits = O.cached_decode_reference(ids, p, cfg, 5, dtype=D64)
    assert torch.equal(toks, full[:, 7:])
    forced = torch.randint(0, 61, (3, 5), generator=g(44))
    ftoks, flog = O.cached_decode_reference(ids, p, cfg, 5, forced=forced, dtype=D64)
    seq = torch.cat([ids, forced], dim=1)
    for t in range(5):
        e, _ = O.model_forward_reference(seq[:, :7 + t], p, cfg, dtype=D64)
        torch.testing.assert_close(flog[:, t], e[:, -1], rtol=1e-10, atol=1e-10)
        assert torch.equal(ftoks[:, t], O.argmax_lowest_reference(e[:, -1]))


def test_decoder_layer_rounding_points():
    """``rounding`` stores each op's output in that type: float32 storage is the unrounded layer bit
    for bit; bf16 storage gives a bf16-representable output close to the fp32 one, and its error
    grows when the stored activations are coarser (fp16 -> bf16)."""
    cfg = O.OracleConfig(vocab_size=16, hidden_size=64, intermediate_size=96, num_hidden_layers=1,
                         num_attention_heads=4, num_key_value_heads=2, head_dim=16)
    p = O.init_params(cfg, seed=1, std=0.1)
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(2, 9, 64, generator=gen)
    cos, sin = O.rotary_tables_reference(torch.arange(9)[None].expand(2, 9), O.rope_inv_freq(1e6, 16))
    y = O.decoder_layer_reference(x, p, "model.layers.0.", cfg, cos, sin)
    assert torch.equal(O.decoder_layer_reference(x, p, "model.layers.0.", cfg, cos, sin, rounding=torch.float32), y)
    yb = O.decoder_layer_reference(x, p, "model.layers.0.", cfg, cos, sin, rounding=torch.bfloat16)
    yh = O.decoder_layer_reference(x, p, "model.layers.0.", cfg, cos, sin, rounding=torch.float16)
    assert torch.equal(yb, yb.bfloat16().float())
    eb, eh = float((yb - y).abs().max() / y.abs().max()), float((yh - y).abs().max() / y.abs().max())
    assert 0 < eh < eb < 2e-2
