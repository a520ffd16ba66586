"""Module-level parity: the tiny training step (config #1), a Qwen3-8B-shape decoder layer, and
greedy inference with the KV cache, against the CPU oracle."""
import pytest
import torch

import oracle as O
from _util import cosine, greedy_parity, max_rel, seeded

from qwen3_triton._model import ComputeOptions, TritonQwen3ForCausalLM
from qwen3_triton.components import DecoderLayer
from qwen3_triton.configuration import OptimizationOptions
from qwen3_triton.inference import CapturedGreedyRequest, TritonQwen3Inference
from qwen3_triton.model import PrecisionQwen3ForCausalLM

pytestmark = pytest.mark.gpu


def hf_config(oc, **kw):
    from transformers import Qwen3Config
    return Qwen3Config(vocab_size=oc.vocab_size, hidden_size=oc.hidden_size, intermediate_size=oc.intermediate_size,
                       num_hidden_layers=oc.num_hidden_layers, num_attention_heads=oc.num_attention_heads,
                       num_key_value_heads=oc.num_key_value_heads, head_dim=oc.head_dim, rope_theta=oc.rope_theta,
                       rms_norm_eps=oc.rms_norm_eps, tie_word_embeddings=oc.tie_word_embeddings,
                       max_position_embeddings=4096, initializer_range=0.02, **kw)


TINY = O.OracleConfig()  # config #1: 4 layers, hidden 256, 8/2 heads, head_dim 32, I 688, V 4096, untied


def oracle_grads(params, ids, cfg):
    leaf = {k: v.double().requires_grad_() for k, v in params.items()}
    if cfg.tie_word_embeddings:
        leaf["lm_head.weight"] = leaf["model.embed_tokens.weight"]
    logits, loss = O.model_forward_reference(ids, leaf, cfg, labels=ids, dtype=torch.float64)
    loss.backward()
    return logits.detach(), loss.detach(), {k: v.grad for k, v in leaf.items()}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("precision", [False, True])
def test_tiny_training_step(dtype, precision):
    """Config #1: fwd -> CE -> bwd; logits/loss/every parameter gradient vs the fp64 oracle."""
    print(f"tiny step {dtype} precision={precision}", flush=True)
    params = O.init_params(TINY, seed=0, std=0.02)
    ids = torch.randint(0, TINY.vocab_size, (2, 128), generator=seeded(0))
    if precision:
        model = PrecisionQwen3ForCausalLM(hf_config(TINY), OptimizationOptions(), require_8b_shape=False)
    else:
        model = TritonQwen3ForCausalLM(hf_config(TINY), ComputeOptions())
    model.load_hf_state_dict({k: v.to(dtype) for k, v in params.items()})
    model = model.cuda()
    out = model(ids.cuda(), labels=ids.cuda())
    out.loss.backward()
    rounded = {k: v.to(dtype) for k, v in params.items()}  # the oracle sees the same (rounded) weights
    el, eloss, egrads = oracle_grads(rounded, ids, TINY)
    fwd_tol = 2e-2 if dtype == torch.bfloat16 else 1e-4
    assert max_rel(out.logits, el) <= fwd_tol
    assert abs(float(out.loss) - float(eloss)) <= 1e-3 * float(eloss)
    worst = 1.0
    for name, p in model.named_parameters():
        c = cosine(p.grad, egrads[name])
        worst = min(worst, c)
        assert c >= (0.999 if dtype == torch.bfloat16 else 0.99999), f"{name}: cosine {c}"
    print(f"worst grad cosine {worst:.6f}")


def test_tiny_fused_lm_head_loss_matches_unfused():
    params = O.init_params(TINY, seed=0, std=0.02)
    ids = torch.randint(0, TINY.vocab_size, (2, 128), generator=seeded(1))
    losses = []
    grads = []
    for fused in (False, True):
        m = TritonQwen3ForCausalLM(hf_config(TINY), ComputeOptions(fused_lm_head_loss=fused))
        m.load_hf_state_dict({k: v.to(torch.bfloat16) for k, v in params.items()})
        m = m.cuda()
        out = m(ids.cuda(), labels=ids.cuda())
        out.loss.backward()
        losses.append(float(out.loss))
        grads.append(m.lm_head.weight.grad.float())
    assert abs(losses[0] - losses[1]) <= 1e-3 * losses[0]
    assert cosine(grads[1], grads[0]) >= 0.999


def test_decoder_layer_8b_shape():
    """One Qwen3-8B decoder layer (bf16, fused norm-rope and gate/up) at 256 tokens: output and
    every gradient vs the fp32 oracle."""
    oc = O.OracleConfig(vocab_size=16, hidden_size=4096, intermediate_size=12288, num_hidden_layers=1,
                        num_attention_heads=32, num_key_value_heads=8, head_dim=128)
    gen = seeded(3)
    params = O.init_params(oc, seed=3, std=0.02, dtype=torch.bfloat16)
    layer = DecoderLayer(hf_config(oc), OptimizationOptions())
    layer.load_state_dict({k[len("model.layers.0."):]: v for k, v in params.items()
                           if k.startswith("model.layers.0.")})
    layer = layer.cuda().to(torch.bfloat16)
    x = torch.randn(1, 256, 4096, generator=gen).to(torch.bfloat16)
    dy = torch.randn(1, 256, 4096, generator=gen).to(torch.bfloat16)
    pos = torch.arange(256)[None]
    cos, sin = O.rotary_tables_reference(pos, O.rope_inv_freq(1e6, 128), dtype=torch.bfloat16)
    xd = x.cuda().requires_grad_()
    y = layer(xd, (cos.cuda(), sin.cuda()))
    y.backward(dy.cuda())
    leaf = {k: v.float().requires_grad_() for k, v in params.items() if k.startswith("model.layers.0.")}
    xr = x.float().requires_grad_()
    yr = O.decoder_layer_reference(xr, leaf, "model.layers.0.", oc, cos.float(), sin.float())
    yr.backward(dy.float())
    assert max_rel(y, yr) <= 2e-2
    assert cosine(xd.grad, xr.grad) >= 0.999
    for name, p in layer.named_parameters():
        c = cosine(p.grad, leaf["model.layers.0." + name].grad)
        assert c >= 0.999, f"{name}: {c}"


def test_decoder_layer_fused_residuals_match_composition():
    """The Qwen3-8B decoder layer at 4096 tokens (the full-tile grid, so the o_proj / down_proj GEMMs
    take the residual epilogue and the MLP block its SwiGLU-backward epilogue): output and every
    gradient bit-equal to the same modules composed with separate residual adds."""
    from qwen3_triton.kernels.norm import rms_norm_fork
    from qwen3_triton.kernels.residual import residual_add
    from qwen3_triton.kernels.mlp_precision import gate_up_swiglu
    from qwen3_triton.kernels.linear import linear
    oc = O.OracleConfig(vocab_size=16, hidden_size=4096, intermediate_size=12288, num_hidden_layers=1,
                        num_attention_heads=32, num_key_value_heads=8, head_dim=128)
    torch.manual_seed(5)
    layer = DecoderLayer(hf_config(oc), OptimizationOptions()).cuda().to(torch.bfloat16)
    gen = seeded(5)
    x = torch.randn(2, 2048, 4096, generator=gen).to(torch.bfloat16).cuda()
    dy = torch.randn(2, 2048, 4096, generator=gen).to(torch.bfloat16).cuda()
    pos = torch.arange(2048)[None].expand(2, 2048).contiguous()
    cos, sin = O.rotary_tables_reference(pos, O.rope_inv_freq(1e6, 128), dtype=torch.bfloat16)
    pe = (cos.cuda(), sin.cuda())

    def composed(xi):
        a, m = layer.self_attn, layer.mlp
        xa, h = rms_norm_fork(xi, layer.input_layernorm.weight, layer.input_layernorm.eps)
        xa = residual_add(xa, a(h, pe))
        xb, h = rms_norm_fork(xa, layer.post_attention_layernorm.weight, layer.post_attention_layernorm.eps)
        return residual_add(xb, linear(gate_up_swiglu(h, m.gate_proj.weight, m.up_proj.weight), m.down_proj.weight))

    runs = []
    for fn in (lambda xi: layer(xi, pe), composed):
        layer.zero_grad(set_to_none=True)
        xi = x.clone().requires_grad_()
        y = fn(xi)
        y.backward(dy)
        runs.append([y.detach(), xi.grad] + [p.grad.clone() for p in layer.parameters()])
    for i, (a, b) in enumerate(zip(*runs)):
        assert torch.equal(a, b), i


SMALL = O.OracleConfig(vocab_size=1000, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=128)


def small_model(seed=4):
    params = O.init_params(SMALL, seed=seed, std=0.05, dtype=torch.bfloat16)
    model = TritonQwen3Inference(hf_config(SMALL))
    model.load_hf_state_dict(params)
    return model.to("cuda"), params


@pytest.mark.parametrize("b,s", [(1, 16), (2, 33), (8, 9)])
def test_prefill_and_cached_decode_logits(b, s):
    model, params = small_model()
    ids = torch.randint(0, SMALL.vocab_size, (b, s + 3), generator=seeded(s))
    cache = model.new_cache(b, s + 3)
    lg = model(ids[:, :s].cuda(), past_key_values=cache, logits_to_keep=s).logits
    el, _ = O.model_forward_reference(ids[:, :s], params, SMALL)
    assert max_rel(lg, el) <= 2e-2
    for t in range(3):   # one token at a time through the KV cache
        lg = model(ids[:, s + t:s + t + 1].cuda(), past_key_values=cache).logits
        el, _ = O.model_forward_reference(ids[:, :s + t + 1], params, SMALL)
        assert max_rel(lg[:, 0], el[:, -1]) <= 2e-2
    assert cache.length == s + 3


@pytest.mark.parametrize("b,s", [(1, 12), (3, 7)])
def test_greedy_tokens_vs_oracle(b, s):
    """Greedy tokens vs the fp32 oracle on the same bf16 weights: teacher-forced logits and every
    decisive step's token (margin above twice the measured logit error), at least 75 % of the steps
    decisive, then the free-running tokens up to each row's first non-decisive step."""
    model, params = small_model(seed=5)
    ids = torch.randint(0, SMALL.vocab_size, (b, s), generator=seeded(7))
    greedy_parity(model, {k: v.float() for k, v in params.items()}, SMALL, ids, 8, label=f"small B{b}")


@pytest.mark.parametrize("budget", [1, 40])
def test_captured_request_budgets(budget):
    """The captured request is two fixed-size graphs (prefill, one decode step) whatever the budget:
    a 1-token budget (prefill graph only) and a 40-token one reproduce the eager loop."""
    model, _ = small_model(seed=6)
    ids = torch.randint(0, SMALL.vocab_size, (3, 21), generator=seeded(18)).cuda()
    eager = model.generate(ids, max_new_tokens=budget, eos_token_id=[], pad_token_id=0)
    req = CapturedGreedyRequest(model, ids, max_new_tokens=budget)
    for _ in range(2):
        out = req(ids).clone()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_captured_request_replays_eager_tokens():
    model, _ = small_model(seed=6)
    ids = torch.randint(0, SMALL.vocab_size, (2, 10), generator=seeded(8)).cuda()
    eager = model.generate(ids, max_new_tokens=5, eos_token_id=[], pad_token_id=0)
    req = CapturedGreedyRequest(model, ids, max_new_tokens=5)
    for _ in range(3):
        torch.cuda.synchronize()
        assert torch.equal(req(ids).clone(), eager)
    other = torch.randint(0, SMALL.vocab_size, (2, 10), generator=seeded(9)).cuda()
    assert torch.equal(req(other).clone(), model.generate(other, max_new_tokens=5, eos_token_id=[], pad_token_id=0))


def test_generate_eos_and_padding():
    model, _ = small_model(seed=6)
    ids = torch.randint(0, SMALL.vocab_size, (2, 10), generator=seeded(8)).cuda()
    free = model.generate(ids, max_new_tokens=4, eos_token_id=[], pad_token_id=0)
    eos = int(free[0, 11])  # row 0's second generated token becomes EOS
    out = model.generate(ids, max_new_tokens=4, eos_token_id=[eos], pad_token_id=7)
    assert out[0, 11] == eos
    assert bool((out[0, 12:] == 7).all())


@pytest.mark.parametrize("b,s", [(1, 12), (2, 7)])
def test_decode_session_replays_one_step_graph(b, s):
    """One captured decode step replayed at every position (device-resident cache length) gives the
    same tokens as the eager generate loop."""
    from qwen3_triton.inference import DecodeSession
    model, _ = small_model(seed=6)
    ids = torch.randint(0, SMALL.vocab_size, (b, s), generator=seeded(10)).cuda()
    n = 6
    eager = model.generate(ids, max_new_tokens=n, eos_token_id=[], pad_token_id=0)
    sess = DecodeSession(model, b, s + n + 2)
    sess.prefill(ids)
    sess.step()          # eager step
    sess.capture()
    for _ in range(n - 2):
        sess.step()      # replays
    torch.cuda.synchronize()
    assert sess.cache.length == s + n - 1
    assert torch.equal(sess.tokens(), eager)


@pytest.mark.timeout(900)
def test_decoder_layer_8b_benchmark_shape():
    """Config #4's decoder layer exactly as the benchmark times it (B4 x S2048 = 8192 tokens, bf16
    weights N(0, 0.02) and N(0, 1) input / upstream gradient from the device generator, seed 3):
    output (bf16 gate) and every gradient (cosine >= 0.999) against the fp32 host oracle
    (``_model.py:60-108``, ``components.py:18-54``).  At this size every GEMM runs its full-grid
    plan (the residual, SwiGLU and SwiGLU-backward epilogues, the split-M remainder launch of the
    Q/K/V weight gradient) and the weight gradients contract over K = 8192 tokens."""
    oc = O.OracleConfig(vocab_size=16, hidden_size=4096, intermediate_size=12288, num_hidden_layers=1,
                        num_attention_heads=32, num_key_value_heads=8, head_dim=128)
    print("decoder layer B4 S2048 fwd+bwd vs the fp32 oracle (seed 3)", flush=True)
    torch.manual_seed(3)
    layer = DecoderLayer(hf_config(oc), OptimizationOptions()).to(device="cuda", dtype=torch.bfloat16)
    gen = torch.Generator(device="cuda").manual_seed(3)
    with torch.no_grad():
        for name, p in layer.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.normal_(0.0, 0.02, generator=gen)
    b, s = 4, 2048
    x = torch.randn(b, s, 4096, device="cuda", dtype=torch.bfloat16, generator=gen)
    dy = torch.randn(b, s, 4096, device="cuda", dtype=torch.bfloat16, generator=gen)
    pos = torch.arange(s)[None].expand(b, s).contiguous()
    cos, sin = O.rotary_tables_reference(pos, O.rope_inv_freq(1e6, 128), dtype=torch.bfloat16)
    xd = x.clone().requires_grad_()
    y = layer(xd, (cos.cuda(), sin.cuda()))
    y.backward(dy)
    torch.cuda.synchronize()
    leaf = {"model.layers.0." + n: p.detach().float().cpu().requires_grad_() for n, p in layer.named_parameters()}
    xr = x.float().cpu().requires_grad_()
    yr = O.decoder_layer_reference(xr, leaf, "model.layers.0.", oc, cos.float(), sin.float())
    yr.backward(dy.float().cpu())
    rel = max_rel(y, yr)
    cos_x = cosine(xd.grad, xr.grad)
    worst = ("x", cos_x)
    assert rel <= 2e-2, f"y max-rel {rel:.3e}"
    assert cos_x >= 0.999, f"dx cosine {cos_x}"
    for name, p in layer.named_parameters():
        c = cosine(p.grad, leaf["model.layers.0." + name].grad)
        worst = min(worst, (name, c), key=lambda t: t[1])
        assert c >= 0.999, f"{name}: {c}"
    print(f"B4 S2048 layer: y max-rel {rel:.3e}, worst gradient cosine {worst[1]:.6f} ({worst[0]})", flush=True)
