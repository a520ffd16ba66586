"""Trainable Qwen3 graph on the HIP operator set.

Mirrors ``qwen3_triton/_model.py:22-134`` of the reference: the same module classes, parameter
names (official Qwen3 names, so HF state dicts load directly), initialisation, validation and
forward contracts.  Dense, unpadded causal training; no KV cache, sliding window, dropout, RoPE
scaling or attention bias.  Unsupported features fail explicitly.

Layout choice: Q/K/V stay in the projection layout [B,S,H,D]; the flash kernels take their
strides directly, so the reference's transpose(1,2).contiguous() copies are not needed.
"""
from dataclasses import dataclass

import torch
from torch import nn

from ._checkpoint import check_architecture, resolve_tied, rope_theta, scaled_rope  # noqa: F401
from .kernels import _ops
from .kernels.activation import swiglu
from .kernels.attention import causal_attention_bshd
from .kernels.embedding import embedding
from .kernels.linear import linear
from .kernels.lm_head_ce import lm_head_cross_entropy
from .kernels.loss import causal_cross_entropy
from .kernels.norm import rms_norm, rms_norm_fork
from .kernels.residual import residual_add
from .kernels.rotary import apply_rotary, rotary_tables


@dataclass(frozen=True)
class ComputeOptions:
    """Switches of ``_model.py:22-27``; ``fused_lm_head_loss`` (new) computes the loss with the
    vocabulary-chunked LM head + CE and returns no logits."""
    linear_optimized: bool = False
    attention_optimized: bool = False
    loss_optimized: bool = False
    fused_lm_head_loss: bool = False


class TritonLinear(nn.Module):
    def __init__(self, in_features, out_features, std, options):
        super().__init__()
        self.weight = nn.Parameter(torch.empty(out_features, in_features))
        nn.init.normal_(self.weight, std=std)
        self.options = options

    def forward(self, x):
        return linear(x, self.weight, optimized=self.options.linear_optimized)


class TritonEmbedding(nn.Module):
    def __init__(self, vocab, hidden, std):
        super().__init__()
        self.weight = nn.Parameter(torch.empty(vocab, hidden))
        nn.init.normal_(self.weight, std=std)

    def forward(self, ids):
        return embedding(ids, self.weight)


class TritonNorm(nn.Module):
    def __init__(self, hidden, eps):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden))
        self.eps = eps

    def forward(self, x):
        return rms_norm(x, self.weight, self.eps)


class TritonRotary(nn.Module):
    def __init__(self, config):
        super().__init__()
        # Frequencies are static configuration: built on the host in fp32 (``_model.py:49-55``).
        freq = 1. / (rope_theta(config) ** (torch.arange(0, config.head_dim, 2, device='cpu',
                                                         dtype=torch.float32) / config.head_dim))
        self.register_buffer('inv_freq', freq, persistent=False)

    def forward(self, positions, dtype):
        freq = self.inv_freq if self.inv_freq.dtype == torch.float32 else _ops.cast(self.inv_freq, torch.float32)
        return rotary_tables(positions, freq, dtype)


class TritonAttention(nn.Module):
    def __init__(self, c, options):
        super().__init__()
        self.options = options
        self.head_dim = c.head_dim
        self.num_heads = c.num_attention_heads
        self.num_kv_heads = c.num_key_value_heads
        h, std = c.hidden_size, c.initializer_range
        self.q_proj = TritonLinear(h, self.num_heads * self.head_dim, std, options)
        self.k_proj = TritonLinear(h, self.num_kv_heads * self.head_dim, std, options)
        self.v_proj = TritonLinear(h, self.num_kv_heads * self.head_dim, std, options)
        self.o_proj = TritonLinear(self.num_heads * self.head_dim, h, std, options)
        self.q_norm = TritonNorm(self.head_dim, c.rms_norm_eps)
        self.k_norm = TritonNorm(self.head_dim, c.rms_norm_eps)

    def forward(self, x, positions):
        b, s, _ = x.shape
        d = self.head_dim
        cos, sin = positions
        q = self.q_norm(self.q_proj(x).view(b, s, self.num_heads, d))
        k = self.k_norm(self.k_proj(x).view(b, s, self.num_kv_heads, d))
        v = self.v_proj(x).view(b, s, self.num_kv_heads, d)
        q, k = apply_rotary(q, cos, sin), apply_rotary(k, cos, sin)
        y = causal_attention_bshd(q, k, v, scale=d ** -0.5)
        return self.o_proj(y.reshape(b, s, self.num_heads * d))


class TritonMLP(nn.Module):
    def __init__(self, c, options):
        super().__init__()
        h, i, std = c.hidden_size, c.intermediate_size, c.initializer_range
        self.gate_proj = TritonLinear(h, i, std, options)
        self.up_proj = TritonLinear(h, i, std, options)
        self.down_proj = TritonLinear(i, h, std, options)

    def forward(self, x):
        return self.down_proj(swiglu(self.gate_proj(x), self.up_proj(x)))


class TritonDecoderLayer(nn.Module):
    def __init__(self, c, options):
        super().__init__()
        self.self_attn = TritonAttention(c, options)
        self.mlp = TritonMLP(c, options)
        self.input_layernorm = TritonNorm(c.hidden_size, c.rms_norm_eps)
        self.post_attention_layernorm = TritonNorm(c.hidden_size, c.rms_norm_eps)

    def forward(self, x, position_embeddings):
        # x feeds both the residual sum and the norm: one fork node, so the backward sums the two
        # gradients of x inside the RMSNorm backward kernel (``_model.py:60-108`` layer order).
        x, h = rms_norm_fork(x, self.input_layernorm.weight, self.input_layernorm.eps)
        x = residual_add(x, self.self_attn(h, position_embeddings))
        x, h = rms_norm_fork(x, self.post_attention_layernorm.weight, self.post_attention_layernorm.eps)
        return residual_add(x, self.mlp(h))


class TritonQwen3Model(nn.Module):
    decoder_class = TritonDecoderLayer

    def __init__(self, c, options):
        super().__init__()
        self.embed_tokens = TritonEmbedding(c.vocab_size, c.hidden_size, c.initializer_range)
        self.layers = nn.ModuleList([self.decoder_class(c, options) for _ in range(c.num_hidden_layers)])
        self.norm = TritonNorm(c.hidden_size, c.rms_norm_eps)
        self.rotary_emb = TritonRotary(c)

    def forward(self, ids, position_ids=None):
        x = self.embed_tokens(ids)
        positions = self.rotary_emb(self._positions_for(ids, position_ids), x.dtype)
        for layer in self.layers:
            x = layer(x, positions)
        return self.norm(x)

    @staticmethod
    def _positions_for(ids, position_ids):
        """[B, S] int64 positions: 0..S-1 per row by default; one [1, S] row is shared by the batch."""
        b, s = ids.shape
        if position_ids is None:
            return _ops.positions(b, s, 0, ids.device)
        if tuple(position_ids.shape) == (1, s) and b > 1:
            position_ids = position_ids.expand(b, s).contiguous()
        if tuple(position_ids.shape) != (b, s):
            raise ValueError(f'position_ids of shape {tuple(position_ids.shape)} do not match input_ids {(b, s)}')
        return position_ids


class TritonQwen3ForCausalLM(nn.Module):
    backbone_class = TritonQwen3Model
    # HF forward features this dense causal-training model does not provide (no silent fallback).
    _UNSUPPORTED_FORWARD = ('use_cache', 'past_key_values', 'attention_mask', 'output_attentions',
                            'output_hidden_states', 'logits_to_keep')

    def __init__(self, config, options=None):
        super().__init__()
        check_architecture(config)
        self.config = config
        self.options = options or ComputeOptions()
        self.model = self.backbone_class(config, self.options)
        self.lm_head = TritonLinear(config.hidden_size, config.vocab_size, config.initializer_range, self.options)
        self.tie_weights()

    def tie_weights(self):
        """Share the embedding matrix as the LM head when the config ties them."""
        if self.config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight

    def load_hf_state_dict(self, state, *, assign=False):
        """Load official Qwen3 parameter names (strict); a tied checkpoint may omit the LM head."""
        result = self.load_state_dict(resolve_tied(state, self.config.tie_word_embeddings), strict=True,
                                      assign=assign)
        self.tie_weights()
        return result

    def forward(self, input_ids, labels=None, *, position_ids=None, use_cache=False, attention_mask=None,
                past_key_values=None, output_attentions=False, output_hidden_states=False, return_dict=True,
                logits_to_keep=0):
        from transformers.modeling_outputs import CausalLMOutputWithPast
        asked = dict(use_cache=use_cache, past_key_values=past_key_values is not None,
                     attention_mask=attention_mask is not None, output_attentions=output_attentions,
                     output_hidden_states=output_hidden_states, logits_to_keep=logits_to_keep)
        requested = [k for k in self._UNSUPPORTED_FORWARD if asked[k]]
        if requested:
            raise ValueError(f'dense unpadded causal training only; not implemented: {", ".join(requested)}')
        if input_ids.ndim != 2 or input_ids.dtype not in (torch.int32, torch.int64):
            raise ValueError('input_ids must be an integer [batch, sequence] tensor')
        hidden = self.model(input_ids, position_ids)
        logits = loss = None
        if labels is not None and self.options.fused_lm_head_loss:
            loss = lm_head_cross_entropy(hidden, self.lm_head.weight, labels)
        else:
            logits = self.lm_head(hidden)
            if labels is not None:
                loss = causal_cross_entropy(logits, labels, optimized=self.options.loss_optimized)
        if return_dict:
            return CausalLMOutputWithPast(loss=loss, logits=logits)
        return (logits,) if labels is None else (loss, logits)
