"""Config #5 at Qwen3-8B width: prefill + KV-cached greedy decode against the fp32 oracle.

Qwen3-8B's per-layer shapes and vocabulary (hidden 4096, 32 query / 8 KV heads, head_dim 128,
intermediate 12288, vocabulary 151936, untied LM head) with 2 of the 36 layers, random bf16
weights N(0, 0.02) from seed 4 (norm weights 1), as in the benchmark's synthetic model.  The oracle
runs in fp32 on the host with the same bf16-rounded weights (``inference/model.py:102-188``).
"""
import pytest
import torch

import oracle as O
from _util import greedy_parity, max_rel, seeded

from qwen3_triton.inference import CapturedGreedyRequest, DecodeSession, TritonQwen3Inference

pytestmark = pytest.mark.gpu

CFG = O.OracleConfig(vocab_size=151936, hidden_size=4096, intermediate_size=12288, num_hidden_layers=2,
                     num_attention_heads=32, num_key_value_heads=8, head_dim=128)


def hf_config(oc):
    from transformers import Qwen3Config
    return Qwen3Config(vocab_size=oc.vocab_size, hidden_size=oc.hidden_size, intermediate_size=oc.intermediate_size,
                       num_hidden_layers=oc.num_hidden_layers, num_attention_heads=oc.num_attention_heads,
                       num_key_value_heads=oc.num_key_value_heads, head_dim=oc.head_dim, rope_theta=oc.rope_theta,
                       rms_norm_eps=oc.rms_norm_eps, tie_word_embeddings=False, max_position_embeddings=40960)


@pytest.fixture(scope="module")
def width8b():
    print("building the 2-layer Qwen3-8B-width model (seed 4)", flush=True)
    params = O.init_params(CFG, seed=4, std=0.02, dtype=torch.bfloat16)
    model = TritonQwen3Inference(hf_config(CFG))
    model.load_hf_state_dict({k: v.cuda() for k, v in params.items()})
    p32 = {k: v.float() for k, v in params.items()}
    del params
    yield model, p32
    del model
    torch.cuda.empty_cache()


@pytest.mark.parametrize("b,s", [(1, 128), (8, 64)])
def test_prefill_logits_8b_width(width8b, b, s):
    """Every prefill position's logits (B1 and B8) against the fp32 oracle: bf16 forward gate."""
    model, p32 = width8b
    print(f"config #5 prefill B{b} S{s}", flush=True)
    ids = torch.randint(0, CFG.vocab_size, (b, s), generator=seeded(40 + b))
    cache = model.new_cache(b, s)
    got = model(ids.cuda(), past_key_values=cache, logits_to_keep=s).logits
    exp, _ = O.model_forward_reference(ids, p32, CFG)
    assert max_rel(got, exp) <= 2e-2


@pytest.mark.parametrize("b,s", [(1, 128), (8, 64)])
def test_greedy_decode_8b_width(width8b, b, s):
    """12 greedy steps at B1 / B8: teacher-forced logits and decisive tokens against the oracle, the
    free-running tokens of ``generate``, and the captured one-step graph (``DecodeSession``, the
    benchmark's decode path) reproducing ``generate`` token for token."""
    model, p32 = width8b
    steps = 12
    print(f"config #5 greedy B{b} S{s} x {steps} steps", flush=True)
    ids = torch.randint(0, CFG.vocab_size, (b, s), generator=seeded(50 + b))
    greedy_parity(model, p32, CFG, ids, steps, label=f"8B-width B{b}")
    eager = model.generate(ids.cuda(), max_new_tokens=steps, eos_token_id=[], pad_token_id=0)
    sess = DecodeSession(model, b, s + steps + 1)
    sess.prefill(ids.cuda())
    sess.capture()
    for _ in range(steps - 1):
        sess.step()
    torch.cuda.synchronize()
    assert torch.equal(sess.tokens(), eager)
    req = CapturedGreedyRequest(model, ids.cuda(), max_new_tokens=steps)   # two fixed-size graphs
    assert torch.equal(req(ids.cuda()).clone(), eager)
