"""Qwen3 configuration checks and checkpoint reading shared by the training and inference models.

Covers what ``qwen3_triton/_model.py:112-126`` and ``qwen3_triton/inference/model.py:59-88`` do
on the reference side -- refuse architectures the kernels do not implement, resolve tied input /
output embeddings, read a local (optionally sharded) safetensors checkpoint -- organised as one
checked rule table, one tie resolver and one shard walker.  Only names, parameter keys and the
exception types (``ValueError`` for a bad configuration or checkpoint) are fixed by the reference.
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

EMBED = 'model.embed_tokens.weight'
HEAD = 'lm_head.weight'


def rope_theta(config):
    """RoPE base of an HF Qwen3 config (``rope_theta``, or ``rope_parameters['rope_theta']`` in
    newer transformers releases)."""
    theta = getattr(config, 'rope_theta', None)
    if theta is None:
        theta = (getattr(config, 'rope_parameters', None) or {}).get('rope_theta', 10000.0)
    return float(theta)


def scaled_rope(config):
    """True when the config asks for a RoPE scaling variant (anything but the plain rotation)."""
    for name in ('rope_scaling', 'rope_parameters'):
        spec = getattr(config, name, None)
        if spec and spec.get('rope_type', spec.get('type', 'default')) not in (None, 'default'):
            return True
    return False


# Each rule: (violated?, what the kernels do not implement).  Checked in order; the first violation raises.
_ARCHITECTURE_RULES = (
    (lambda c: c.model_type != 'qwen3', 'model_type must be "qwen3"'),
    (lambda c: c.hidden_act != 'silu', 'only the SiLU (SwiGLU) MLP is implemented'),
    (lambda c: c.attention_dropout != 0, 'attention dropout is not implemented'),
    (lambda c: bool(getattr(c, 'attention_bias', False)), 'attention projections have no bias here'),
    (lambda c: bool(getattr(c, 'use_sliding_window', False)), 'sliding-window attention is not implemented'),
    (scaled_rope, 'scaled RoPE variants are not implemented'),
    (lambda c: c.head_dim % 2 != 0, 'the rotary head dimension must be even'),
    (lambda c: c.num_attention_heads % c.num_key_value_heads != 0,
     'query heads must be a multiple of key/value heads (GQA)'),
)


def check_architecture(config):
    """Raise ValueError naming the first feature of ``config`` the HIP kernels do not implement."""
    for violated, what in _ARCHITECTURE_RULES:
        if violated(config):
            raise ValueError(f'unsupported Qwen3 configuration: {what}')


def resolve_tied(state, tied):
    """A copy of the HF state dict with the LM head filled in from the embedding when ``tied``.

    A tied checkpoint may omit ``lm_head.weight``; if it carries one, it must equal the embedding."""
    state = dict(state)
    if not tied:
        return state
    if EMBED not in state:
        raise ValueError(f'checkpoint lacks {EMBED}')
    head = state.setdefault(HEAD, state[EMBED])
    if head is not state[EMBED] and not torch.equal(head, state[EMBED]):
        raise ValueError('tie_word_embeddings is set but the checkpoint\'s lm_head.weight differs from '
                         'model.embed_tokens.weight')
    return state


def shard_files(root):
    """The safetensors files of a local checkpoint directory: the distinct shards named by
    ``model.safetensors.index.json`` (sorted), else ``model.safetensors``.  A shard path that
    resolves outside ``root`` (``..`` or an absolute name in the index) is refused."""
    root = Path(root).resolve()
    index = root / 'model.safetensors.index.json'
    names = sorted(set(json.loads(index.read_text())['weight_map'].values())) if index.is_file() \
        else ['model.safetensors']
    files = []
    for name in names:
        f = (root / name).resolve()
        if root not in f.parents:
            raise ValueError(f'checkpoint shard {name!r} lies outside {root}')
        if not f.is_file():
            raise FileNotFoundError(f'checkpoint shard {f} is missing')
        files.append(f)
    return files


def read_checkpoint(root, device='cpu'):
    """Every tensor of a local safetensors checkpoint, read shard by shard straight onto ``device``
    (no whole-model host copy when ``device`` is a GPU)."""
    from safetensors import safe_open
    dev = str(torch.device(device))
    state = {}
    for f in shard_files(root):
        with safe_open(str(f), framework='pt', device=dev) as reader:
            for key in reader.keys():
                if key in state:
                    raise ValueError(f'tensor {key!r} appears in more than one shard')
                state[key] = reader.get_tensor(key)
    return state
