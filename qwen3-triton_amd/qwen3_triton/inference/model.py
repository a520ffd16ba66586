"""Dense bf16 Qwen3 inference: single device, unpadded equal-length batches, contiguous KV cache,
greedy decoding.  Mirrors ``qwen3_triton/inference/model.py:26-225`` (``KVCache``,
``TritonQwen3Inference``, ``CapturedGreedyRequest``); the arithmetic is the HIP kernels.
"""
from dataclasses import dataclass
from pathlib import Path

import torch
from torch import nn

from .._model import TritonQwen3ForCausalLM, rope_theta
from ..configuration import OptimizationOptions
from ..kernels import _ops
from ..kernels.activation import swiglu
from ..kernels.embedding import embedding
from ..kernels.mlp_precision import gate_up_swiglu
from ..kernels.residual import residual_add
from . import kernels


@dataclass
class KVCache:
    """Request-owned [layer][batch, KV-head, capacity, head-dim] storage (``inference/model.py:26-45``).

    Only positions below ``length`` are readable; reset keeps the allocation and discards the
    logical contents.  A failed forward invalidates the cache until an explicit reset."""
    keys: list
    values: list
    capacity: int
    batch_size: int
    owner: object
    length: int = 0
    valid: bool = True

    @property
    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in self.keys + self.values)

    def reset(self):
        self.length = 0
        self.valid = True


class TritonQwen3Inference(nn.Module):
    def __init__(self, config, *, gemv=True, split_decode=False, sliced_decode=False, prefill_tiling=False,
                 reference_accumulation=False):
        super().__init__()
        if config.head_dim != 128:
            raise ValueError('The qualified Qwen3 attention head dimension is 128')
        with torch.device('meta'):
            core = TritonQwen3ForCausalLM(config, OptimizationOptions())
        self.model = core.model
        self.lm_head = core.lm_head
        self.config = config
        self.gemv, self.split_decode = gemv, split_decode
        self._cache_owner = object()
        try:
            from transformers import GenerationConfig
            self.generation_config = GenerationConfig.from_model_config(config)
        except Exception:  # pragma: no cover - generation defaults only
            self.generation_config = None
        self.eval()

    # ------------------------------------------------------------------ weights
    def load_hf_state_dict(self, state):
        state = dict(state)
        if self.config.tie_word_embeddings and 'lm_head.weight' not in state:
            state['lm_head.weight'] = state['model.embed_tokens.weight']
        if self.config.tie_word_embeddings and not torch.equal(state['lm_head.weight'],
                                                               state['model.embed_tokens.weight']):
            raise ValueError('Tied checkpoint weights disagree')
        self.load_state_dict(state, assign=True, strict=True)
        if self.config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight
        if any(p.dtype != torch.bfloat16 for p in self.parameters()):
            raise ValueError('BF16 inference checkpoint required')
        self.model.rotary_emb.inv_freq = self._inv_freq()
        return self

    def _inv_freq(self):
        c = self.config
        return 1. / (rope_theta(c) ** (torch.arange(0, c.head_dim, 2, dtype=torch.float32) / c.head_dim))

    @classmethod
    def random_init(cls, config, *, seed=0, std=0.02, device='cuda', **kw):
        """Random N(0, std) bf16 weights (norm weights 1), generated directly on ``device``: the
        benchmark's synthetic 8B model without a host copy."""
        model = cls(config, **kw)
        gen = torch.Generator(device=device).manual_seed(seed)
        state = {}
        for name, p in model.named_parameters():
            if name.endswith('norm.weight'):
                state[name] = torch.ones(p.shape, dtype=torch.bfloat16, device=device)
            else:
                t = torch.empty(p.shape, dtype=torch.bfloat16, device=device)
                t.normal_(0.0, std, generator=gen)
                state[name] = t
        model.load_hf_state_dict(state)
        model.model.rotary_emb.inv_freq = model.model.rotary_emb.inv_freq.to(device)
        return model

    @classmethod
    def from_pretrained(cls, path, *, device='cuda', **kw):
        """Load local official safetensors (``inference/model.py:68-88``); no download."""
        import json
        from safetensors import safe_open
        from transformers import AutoConfig
        path = Path(path).resolve()
        config = AutoConfig.from_pretrained(path, local_files_only=True)
        model = cls(config, **kw)
        index = path / 'model.safetensors.index.json'
        shards = sorted(set(json.loads(index.read_text())['weight_map'].values())) if index.exists() \
            else ['model.safetensors']
        state = {}
        for name in shards:
            shard = (path / name).resolve()
            if not shard.is_relative_to(path):
                raise ValueError('Checkpoint shard escapes model directory')
            with safe_open(shard, framework='pt', device='cpu') as f:
                for key in f.keys():
                    state[key] = f.get_tensor(key)
        model.load_hf_state_dict(state)
        del state
        model.to(device=device)
        return model

    @property
    def device(self):
        return self.lm_head.weight.device

    def new_cache(self, batch_size, max_length):
        if type(batch_size) is not int or batch_size < 1 or type(max_length) is not int or \
                not 1 <= max_length <= self.config.max_position_embeddings:
            raise ValueError('Positive batch/capacity within max_position_embeddings required')
        if self.device.type != 'cuda':
            raise ValueError('Load BF16 weights onto a ROCm device first')
        shape = (batch_size, self.config.num_key_value_heads, max_length, self.config.head_dim)
        keys = [torch.empty(shape, device=self.device, dtype=torch.bfloat16) for _ in self.model.layers]
        values = [torch.empty(shape, device=self.device, dtype=torch.bfloat16) for _ in self.model.layers]
        return KVCache(keys, values, max_length, batch_size, self._cache_owner)

    # ------------------------------------------------------------------ forward
    def _forward(self, input_ids, cache, logits_to_keep, *, validate_ids=True, start_dev=None):
        from transformers.modeling_outputs import CausalLMOutputWithPast
        if input_ids.ndim != 2 or input_ids.dtype not in (torch.int32, torch.int64) or \
                input_ids.device != self.device or not input_ids.is_contiguous():
            raise ValueError('Contiguous integer ROCm [B,S] input_ids on model device required')
        b, s = input_ids.shape
        if b < 1 or s < 1:
            raise ValueError('Nonempty batch/sequence required')
        if cache.owner is not self._cache_owner or not cache.valid or b != cache.batch_size or \
                cache.length + s > cache.capacity:
            raise ValueError('Foreign, invalid, mismatched or exhausted KV cache')
        if type(logits_to_keep) is not int or not 0 <= logits_to_keep <= s:
            raise ValueError('logits_to_keep must be 0 or within current sequence length')
        if validate_ids and not bool(((input_ids >= 0) & (input_ids < self.config.vocab_size)).all()):
            raise ValueError('Token ID outside vocabulary')
        start = cache.length
        if start_dev is not None and s != 1:
            raise ValueError('device-resident positions are for single-token decode steps')
        pos = kernels.positions(b, s, start, self.device, start_dev)
        try:
            x = embedding(input_ids, self.model.embed_tokens.weight)
            cos, sin = self.model.rotary_emb(pos, torch.bfloat16)
            fused = self.gemv and kernels.decode_linear_ok(x, self.lm_head.weight)
            for i, layer in enumerate(self.model.layers):
                a = layer.self_attn
                d = a.head_dim
                if fused:  # decode step: norms, residual adds and SwiGLU ride in the projections
                    q, k, v = kernels.decode_linear(x, [a.q_proj.weight, a.k_proj.weight, a.v_proj.weight],
                                                    norm_weight=layer.input_layernorm.weight,
                                                    eps=layer.input_layernorm.eps)
                    q = q.view(b, s, a.num_heads, d)
                    k = k.view(b, s, a.num_kv_heads, d)
                    v = v.view(b, s, a.num_kv_heads, d)
                    if s == 1 and d == 128 and a.q_norm.eps == a.k_norm.eps:
                        y = kernels.decode_step_attention(q, k, v, a.q_norm.weight, a.k_norm.weight, a.q_norm.eps,
                                                          cos, sin, cache.keys[i], cache.values[i], start,
                                                          start_dev).reshape(b, s, -1)
                    else:
                        q = kernels.norm_rope(q, a.q_norm.weight, cos, sin, a.q_norm.eps)
                        k = kernels.norm_rope(k, a.k_norm.weight, cos, sin, a.k_norm.eps)
                        kernels.append(k, v, cache.keys[i], cache.values[i], start, start_dev)
                        y = kernels.attention(q, cache.keys[i], cache.values[i], start,
                                              split_decode=self.split_decode, start_dev=start_dev).reshape(b, s, -1)
                    x = kernels.decode_linear(y, [a.o_proj.weight], mode=1, res=x)
                    m = layer.mlp
                    y = kernels.decode_linear(x, [m.gate_proj.weight, m.up_proj.weight], mode=2,
                                              norm_weight=layer.post_attention_layernorm.weight,
                                              eps=layer.post_attention_layernorm.eps)
                    x = kernels.decode_linear(y, [m.down_proj.weight], mode=1, res=x)
                    continue
                h = kernels.rms_norm(x, layer.input_layernorm.weight, layer.input_layernorm.eps)
                q = kernels.linear(h, a.q_proj.weight, gemv=self.gemv).view(b, s, a.num_heads, d)
                k = kernels.linear(h, a.k_proj.weight, gemv=self.gemv).view(b, s, a.num_kv_heads, d)
                v = kernels.linear(h, a.v_proj.weight, gemv=self.gemv).view(b, s, a.num_kv_heads, d)
                q = kernels.norm_rope(q, a.q_norm.weight, cos, sin, a.q_norm.eps)
                k = kernels.norm_rope(k, a.k_norm.weight, cos, sin, a.k_norm.eps)
                kernels.append(k, v, cache.keys[i], cache.values[i], start, start_dev)
                y = kernels.attention(q, cache.keys[i], cache.values[i], start, split_decode=self.split_decode,
                                      start_dev=start_dev).reshape(b, s, -1)
                x = residual_add(x, kernels.linear(y, a.o_proj.weight, gemv=self.gemv))
                h = kernels.rms_norm(x, layer.post_attention_layernorm.weight, layer.post_attention_layernorm.eps)
                m = layer.mlp
                if b * s <= 8 and self.gemv:
                    y = swiglu(kernels.linear(h, m.gate_proj.weight, gemv=True),
                               kernels.linear(h, m.up_proj.weight, gemv=True))
                else:
                    y = gate_up_swiglu(h, m.gate_proj.weight, m.up_proj.weight, optimized=True)
                x = residual_add(x, kernels.linear(y, m.down_proj.weight, gemv=self.gemv))
            if logits_to_keep:
                x = x[:, -logits_to_keep:, :].contiguous()
            if fused:
                logits = kernels.decode_linear(x, [self.lm_head.weight], norm_weight=self.model.norm.weight,
                                               eps=self.model.norm.eps)[0]
            else:
                x = kernels.rms_norm(x, self.model.norm.weight, self.model.norm.eps)
                logits = kernels.linear(x, self.lm_head.weight, gemv=self.gemv)
            cache.length = start + s
        except BaseException:
            cache.valid = False
            raise
        return CausalLMOutputWithPast(logits=logits, past_key_values=cache)

    @torch.inference_mode()
    def forward(self, input_ids, *, past_key_values=None, use_cache=True, logits_to_keep=1):
        """Append an input chunk; cache.length supplies the absolute RoPE/causal offsets.
        ``use_cache=False`` allows full-sequence recomputation for verification."""
        if not use_cache and past_key_values is not None:
            raise ValueError('A supplied cache requires use_cache=True')
        cache = past_key_values or self.new_cache(input_ids.shape[0], input_ids.shape[1])
        out = self._forward(input_ids, cache, logits_to_keep)
        if not use_cache:
            out.past_key_values = None
        return out

    @torch.inference_mode()
    def generate(self, input_ids, *, max_new_tokens=32, eos_token_id=None, pad_token_id=None):
        """Greedy decoding with per-row EOS, padding and a request-local cache
        (``inference/model.py:158-188``)."""
        if type(max_new_tokens) is not int or max_new_tokens < 0:
            raise ValueError('Nonnegative max_new_tokens required')
        gc = self.generation_config
        eos = (gc.eos_token_id if gc is not None else None) if eos_token_id is None else eos_token_id
        eos = () if eos is None else ((eos,) if isinstance(eos, int) else tuple(eos))
        if any(type(x) is not int or not 0 <= x < self.config.vocab_size for x in eos):
            raise ValueError('Invalid EOS tokens')
        configured_pad = gc.pad_token_id if gc is not None else None
        pad = pad_token_id if pad_token_id is not None else (configured_pad if configured_pad is not None
                                                             else (eos[0] if eos else 0))
        if type(pad) is not int or not 0 <= pad < self.config.vocab_size:
            raise ValueError('Invalid padding token')
        if max_new_tokens == 0:
            if input_ids.ndim != 2 or input_ids.device != self.device or \
                    input_ids.dtype not in (torch.int32, torch.int64) or min(input_ids.shape) < 1:
                raise ValueError('Nonempty integer ROCm [B,S] required')
            if not bool(((input_ids >= 0) & (input_ids < self.config.vocab_size)).all()):
                raise ValueError('Token ID outside vocabulary')
            return input_ids.clone()
        b, s = input_ids.shape
        cache = self.new_cache(b, s + max_new_tokens)
        output = torch.empty((b, s + max_new_tokens), device=self.device, dtype=torch.int64)
        output[:, :s].copy_(input_ids)
        done = torch.zeros((b,), device=self.device, dtype=torch.bool)
        if not torch.cuda.is_current_stream_capturing():
            if not bool(((input_ids >= 0) & (input_ids < self.config.vocab_size)).all()):
                raise ValueError('Token ID outside vocabulary')
        current = input_ids
        step = 0
        for step in range(max_new_tokens):
            logits = self._forward(current, cache, 1, validate_ids=False).logits[:, 0, :]
            current = torch.empty((b, 1), device=self.device, dtype=torch.int64)
            kernels.select(logits, output, current, done, s + step, eos, pad)
            if eos and bool(done.all()):
                break
        return output[:, :s + step + 1].contiguous()


class DecodeSession:
    """Greedy decoding with ONE captured HIP graph for the decode step, replayed at every position.

    The cache length lives in device memory; the position-dependent kernels (positions, KV
    append, split-KV attention, token write) read it when they run and the step ends with a
    device-side increment, so the same graph serves the whole request.  Prefill runs eagerly.
    No counterpart in the reference (its captured request bakes every position into one graph,
    ``inference/model.py:191-225``); the tokens match ``generate``.
    """

    @torch.inference_mode()
    def __init__(self, model, batch, capacity, *, eos=(), pad=0):
        self.model, self.batch, self.capacity = model, batch, capacity
        self.eos, self.pad = tuple(eos), pad
        dev = model.device
        self.cache = model.new_cache(batch, capacity)
        self.ids = torch.zeros((batch, capacity), device=dev, dtype=torch.int64)
        self.current = torch.zeros((batch, 1), device=dev, dtype=torch.int64)
        self.length = torch.zeros((1,), device=dev, dtype=torch.int64)
        self.done = torch.zeros((batch,), device=dev, dtype=torch.bool)
        self.graph = None
        self.prompt_len = 0

    @torch.inference_mode()
    def prefill(self, input_ids):
        b, s = input_ids.shape
        if b != self.batch or s + 1 > self.capacity or self.cache.length:
            raise ValueError('Prompt does not fit this session')
        self.ids[:, :s].copy_(input_ids)
        logits = self.model._forward(input_ids, self.cache, 1).logits[:, 0, :]
        kernels.select(logits, self.ids, self.current, self.done, s, self.eos, self.pad)
        kernels.advance(self.length, s)
        self.prompt_len = s

    def _step(self):
        logits = self.model._forward(self.current, self.cache, 1, validate_ids=False,
                                     start_dev=self.length).logits[:, 0, :]
        kernels.select(logits, self.ids, self.current, self.done, 1, self.eos, self.pad, position_dev=self.length)
        kernels.advance(self.length, 1)

    @torch.inference_mode()
    def capture(self):
        """Record one decode step (nothing runs; the host-side length is restored)."""
        host_len = self.cache.length
        stream = torch.cuda.Stream(device=self.model.device)
        stream.wait_stream(torch.cuda.current_stream())
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=stream):
            self._step()
        torch.cuda.current_stream().wait_stream(stream)
        self.cache.length = host_len

    @torch.inference_mode()
    def step(self):
        if self.cache.length + 1 > self.capacity:
            raise ValueError('KV cache exhausted')
        if self.graph is None:
            self._step()
            return
        self.graph.replay()
        self.cache.length += 1

    def tokens(self):
        """Prompt plus generated tokens so far ([B, cache.length + 1])."""
        return self.ids[:, :self.cache.length + 1]


class CapturedGreedyRequest:
    """A whole greedy request (prefill + fixed token budget, no early EOS) captured as one HIP
    graph (``inference/model.py:191-225``).  Single-stream and non-reentrant; the returned tokens
    alias request storage until the next replay."""

    @torch.inference_mode()
    def __init__(self, model, input_ids, *, max_new_tokens):
        if type(max_new_tokens) is not int or max_new_tokens < 1:
            raise ValueError('Positive fixed token budget required')
        self.model = model
        self.shape = tuple(input_ids.shape)
        self.busy = False
        self.input = input_ids.clone()
        if not bool(((self.input >= 0) & (self.input < model.config.vocab_size)).all()):
            raise ValueError('Token ID outside vocabulary')
        stream = torch.cuda.Stream(device=model.device)
        stream.wait_stream(torch.cuda.current_stream(model.device))
        with torch.cuda.stream(stream):
            for _ in range(2):
                model.generate(self.input, max_new_tokens=max_new_tokens, eos_token_id=[], pad_token_id=0)
        torch.cuda.current_stream(model.device).wait_stream(stream)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=stream):
            self.output = model.generate(self.input, max_new_tokens=max_new_tokens, eos_token_id=[], pad_token_id=0)

    @torch.inference_mode()
    def __call__(self, input_ids):
        if self.busy:
            raise RuntimeError('Concurrent graph request reuse is unsupported')
        if tuple(input_ids.shape) != self.shape or input_ids.device != self.model.device or \
                input_ids.dtype != self.input.dtype:
            raise ValueError('Captured input shape/device/dtype differs')
        self.busy = True
        try:
            if not bool(((input_ids >= 0) & (input_ids < self.model.config.vocab_size)).all()):
                raise ValueError('Token ID outside vocabulary')
            self.input.copy_(input_ids)
            self.graph.replay()
            return self.output
        finally:
            self.busy = False
