"""Local safetensors checkpoints: single-file and sharded-index forms, tied and untied heads, and the
rejections of ``inference/model.py:68-88`` / ``_model.py:122-126`` (path escape, tied mismatch).

The CPU tests load onto the host (no kernel runs); the ``gpu`` test loads onto the GPU and checks
logits against the oracle."""
import json

import pytest
import torch

import oracle as O
from _util import max_rel, seeded

CFG = O.OracleConfig(vocab_size=300, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                     num_attention_heads=2, num_key_value_heads=1, head_dim=128)


def hf_config(oc, tied):
    from transformers import Qwen3Config
    return Qwen3Config(vocab_size=oc.vocab_size, hidden_size=oc.hidden_size, intermediate_size=oc.intermediate_size,
                       num_hidden_layers=oc.num_hidden_layers, num_attention_heads=oc.num_attention_heads,
                       num_key_value_heads=oc.num_key_value_heads, head_dim=oc.head_dim, rope_theta=oc.rope_theta,
                       rms_norm_eps=oc.rms_norm_eps, tie_word_embeddings=tied, max_position_embeddings=512)


def params(tied, seed=11):
    from dataclasses import replace
    return O.init_params(replace(CFG, tie_word_embeddings=tied), seed=seed, std=0.05, dtype=torch.bfloat16)


def write_checkpoint(root, state, tied, *, shards=1, escape=False):
    """config.json + either model.safetensors or ``shards`` files and an index naming them."""
    from safetensors.torch import save_file
    root.mkdir(parents=True, exist_ok=True)
    hf_config(CFG, tied).save_pretrained(root)
    state = {k: v.contiguous().clone() for k, v in state.items()}
    if shards == 1:
        save_file(state, str(root / "model.safetensors"))
        return root
    keys = sorted(state)
    weight_map = {}
    for i in range(shards):
        name = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        part = {k: state[k] for k in keys[i::shards]}
        save_file(part, str(root / name))
        weight_map.update({k: name for k in part})
    if escape:
        (root.parent / "outside.safetensors").write_bytes((root / name).read_bytes())
        weight_map = {k: ("../outside.safetensors" if v == name else v) for k, v in weight_map.items()}
    (root / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    return root


def loaded_state(model):
    return {k: v for k, v in model.state_dict().items()}


@pytest.mark.parametrize("shards", [1, 3])
@pytest.mark.parametrize("tied", [False, True])
def test_from_pretrained_reads_every_tensor(tmp_path, shards, tied):
    from qwen3_triton.inference import TritonQwen3Inference
    p = params(tied)
    state = dict(p)
    if tied:
        del state["lm_head.weight"]   # tied checkpoints usually omit the head
    root = write_checkpoint(tmp_path / "ckpt", state, tied, shards=shards)
    model = TritonQwen3Inference.from_pretrained(root, device="cpu")
    got = loaded_state(model)
    for k, v in p.items():
        assert torch.equal(got[k], v), k
    if tied:
        assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()
    assert model.model.rotary_emb.inv_freq.dtype == torch.float32
    torch.testing.assert_close(model.model.rotary_emb.inv_freq, O.rope_inv_freq(CFG.rope_theta, CFG.head_dim))


def test_tied_checkpoint_with_different_head_is_rejected(tmp_path):
    from qwen3_triton.inference import TritonQwen3Inference
    state = dict(params(True))
    state["lm_head.weight"] = state["model.embed_tokens.weight"] + 1
    root = write_checkpoint(tmp_path / "ckpt", state, True)
    with pytest.raises(ValueError, match="tie_word_embeddings"):
        TritonQwen3Inference.from_pretrained(root, device="cpu")


def test_shard_outside_the_directory_is_rejected(tmp_path):
    from qwen3_triton.inference import TritonQwen3Inference
    root = write_checkpoint(tmp_path / "ckpt", params(False), False, shards=2, escape=True)
    with pytest.raises(ValueError, match="outside"):
        TritonQwen3Inference.from_pretrained(root, device="cpu")


def test_non_bf16_checkpoint_is_rejected(tmp_path):
    from qwen3_triton.inference import TritonQwen3Inference
    root = write_checkpoint(tmp_path / "ckpt", {k: v.float() for k, v in params(False).items()}, False)
    with pytest.raises(ValueError, match="bf16"):
        TritonQwen3Inference.from_pretrained(root, device="cpu")


def test_training_model_loads_the_same_checkpoint(tmp_path):
    """``TritonQwen3ForCausalLM.load_hf_state_dict`` on a read checkpoint: strict names, the tied head
    filled in, a mismatched tied pair refused."""
    from qwen3_triton._checkpoint import read_checkpoint
    from qwen3_triton._model import TritonQwen3ForCausalLM
    p = params(True)
    state = {k: v for k, v in p.items() if k != "lm_head.weight"}
    root = write_checkpoint(tmp_path / "ckpt", state, True, shards=2)
    model = TritonQwen3ForCausalLM(hf_config(CFG, True))
    model.load_hf_state_dict(read_checkpoint(root))
    assert torch.equal(model.lm_head.weight.detach(), p["model.embed_tokens.weight"])
    bad = dict(state, **{"lm_head.weight": p["model.embed_tokens.weight"] * 2})
    with pytest.raises(ValueError):
        model.load_hf_state_dict(bad)
    with pytest.raises(RuntimeError):      # strict: a missing tensor is an error
        model.load_hf_state_dict({k: v for k, v in state.items() if "q_proj" not in k})


@pytest.mark.gpu
@pytest.mark.parametrize("tied", [False, True])
def test_loaded_checkpoint_logits_vs_oracle(tmp_path, tied):
    """A sharded checkpoint read straight onto the GPU gives the oracle's logits (prefill, all
    positions) and greedy tokens continue from it."""
    from dataclasses import replace
    from qwen3_triton.inference import TritonQwen3Inference
    p = params(tied, seed=12)
    root = write_checkpoint(tmp_path / "ckpt", p, tied, shards=2)
    model = TritonQwen3Inference.from_pretrained(root, device="cuda")
    ids = torch.randint(0, CFG.vocab_size, (2, 24), generator=seeded(13))
    cache = model.new_cache(2, 24)
    got = model(ids.cuda(), past_key_values=cache, logits_to_keep=24).logits
    exp, _ = O.model_forward_reference(ids, p, replace(CFG, tie_word_embeddings=tied))
    assert max_rel(got, exp) <= 2e-2
