"""Dense bf16 Qwen3 inference: single device, unpadded equal-length batches, contiguous KV cache,
greedy decoding.  Mirrors ``qwen3_triton/inference/model.py:26-225`` (``KVCache``,
``TritonQwen3Inference``, ``CapturedGreedyRequest``); the arithmetic is the HIP kernels.
"""
from dataclasses import dataclass
from pathlib import Path

import torch
from torch import nn

from .._checkpoint import read_checkpoint, resolve_tied, rope_theta
from .._model import TritonQwen3ForCausalLM
from ..configuration import OptimizationOptions
from ..kernels import _ops
from ..kernels.activation import swiglu
from ..kernels.embedding import embedding
from ..kernels.linear import (gemm_multi_ok, gemm_nt_multi_into, gemm_nt_residual_into, gemm_nt_residual_norm_into,
                              gemm_residual_ok)
from ..kernels.mlp_precision import gate_up_swiglu
from ..kernels.residual import residual_add
from . import kernels


def _projections(h, weights, gemv):
    """[h W^T for W in weights] for a prefill chunk: one matrix-core launch over the weights side by
    side (``q3_gemm_nt_multi``) where the shapes allow it, else one projection each."""
    m, k = h.numel() // h.shape[-1], h.shape[-1]
    if gemm_multi_ok(h, m, k, weights) and h.is_contiguous() and all(w.is_contiguous() for w in weights):
        outs = [torch.empty((*h.shape[:-1], w.shape[0]), device=h.device, dtype=h.dtype) for w in weights]
        gemm_nt_multi_into(h.view(m, k), weights, [o.view(m, w.shape[0]) for o, w in zip(outs, weights)], m, k)
        return outs
    return [kernels.linear(h, w, gemv=gemv) for w in weights]


def _residual_projection(x, y, weight, gemv, norm=None):
    """x + y W^T, the residual sum in the projection GEMM's epilogue where the shapes allow it.  With
    ``norm`` (an RMSNorm module: the next block's input norm) also returns rms_norm of that sum, formed
    by the GEMM's combining pass where it has one."""
    m, k, n = y.numel() // y.shape[-1], y.shape[-1], weight.shape[0]
    if gemm_residual_ok(y.dtype, m, n, k) and y.is_contiguous() and x.is_contiguous() and weight.is_contiguous():
        out = torch.empty_like(x)
        if norm is not None and n <= 8192 and norm.weight.is_contiguous() and norm.weight.dtype == x.dtype:
            h = torch.empty_like(x)
            gemm_nt_residual_norm_into(y.view(m, k), k, weight, k, x.view(m, n), out.view(m, n), norm.weight,
                                       norm.eps, h.view(m, n), m, n, k)
            return out, h
        gemm_nt_residual_into(y.view(m, k), k, weight, k, x.view(m, n), out.view(m, n), m, n, k)
    else:
        out = residual_add(x, kernels.linear(y, weight, gemv=gemv))
    if norm is None:
        return out
    return out, kernels.rms_norm(out, norm.weight, norm.eps)


@dataclass
class KVCache:
    """Per-request key/value storage, one ``[batch, kv_heads, capacity, head_dim]`` bf16 tensor per
    layer for keys and one for values (the reference's cache fields, ``inference/model.py:26-45``).

    ``length`` positions are filled.  ``reset`` keeps the memory and forgets the contents.  A forward
    that raises marks the cache invalid, and it stays unusable until ``reset``."""
    keys: list
    values: list
    capacity: int
    batch_size: int
    owner: object
    length: int = 0
    valid: bool = True

    @property
    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in (*self.keys, *self.values))

    def reset(self):
        self.length, self.valid = 0, True

    def admit(self, owner, batch, tokens):
        """Raise unless ``tokens`` more positions of ``batch`` rows fit this valid cache of ``owner``."""
        problems = [what for bad, what in (
            (self.owner is not owner, 'belongs to another model'),
            (not self.valid, 'was invalidated by a failed forward (reset it)'),
            (batch != self.batch_size, f'holds batch {self.batch_size}, not {batch}'),
            (self.length + tokens > self.capacity,
             f'has {self.capacity - self.length} free positions, {tokens} needed')) if bad]
        if problems:
            raise ValueError('KV cache ' + '; '.join(problems))


class TritonQwen3Inference(nn.Module):
    def __init__(self, config, *, gemv=True, split_decode=False, sliced_decode=False, prefill_tiling=False,
                 reference_accumulation=False):
        super().__init__()
        if config.head_dim != 128:
            raise ValueError('inference kernels are built for head_dim 128 (the Qwen3 attention head)')
        # The parameters are created on the meta device: a checkpoint or random_init supplies them, so no
        # throw-away initialisation of a multi-GB model happens on the host.
        with torch.device('meta'):
            core = TritonQwen3ForCausalLM(config, OptimizationOptions())
        self.model, self.lm_head, self.config = core.model, core.lm_head, config
        self.gemv, self.split_decode = gemv, split_decode
        self._cache_owner = object()
        self.generation_config = _generation_config(config)
        self.eval()

    # ------------------------------------------------------------------ weights
    def load_hf_state_dict(self, state):
        """Adopt bf16 tensors with official Qwen3 names (strict, no copies: ``assign``)."""
        tied = self.config.tie_word_embeddings
        state = resolve_tied(state, tied)
        wrong = sorted(k for k, v in state.items() if v.dtype != torch.bfloat16 and not k.endswith('inv_freq'))
        if wrong:
            raise ValueError(f'bf16 inference weights required; {wrong[0]} is not bf16')
        self.load_state_dict(state, assign=True, strict=True)
        if tied:
            self.lm_head.weight = self.model.embed_tokens.weight
        self.model.rotary_emb.inv_freq = self._inv_freq().to(self.lm_head.weight.device)
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
        return model.load_hf_state_dict(state)

    @classmethod
    def from_pretrained(cls, path, *, device='cuda', gemv=True, split_decode=False, sliced_decode=False,
                        prefill_tiling=False, reference_accumulation=False):
        """A local Qwen3 safetensors checkpoint (``inference/model.py:68-88``): ``config.json``, an
        optional ``generation_config.json``, and ``model.safetensors`` or the shards named by
        ``model.safetensors.index.json``.  Tensors are read shard by shard straight onto ``device``;
        nothing is downloaded."""
        from transformers import AutoConfig
        path = Path(path).resolve()
        model = cls(AutoConfig.from_pretrained(path, local_files_only=True), gemv=gemv, split_decode=split_decode,
                    sliced_decode=sliced_decode, prefill_tiling=prefill_tiling,
                    reference_accumulation=reference_accumulation)
        if (path / 'generation_config.json').is_file():
            from transformers import GenerationConfig
            model.generation_config = GenerationConfig.from_pretrained(path, local_files_only=True)
        return model.load_hf_state_dict(read_checkpoint(path, device))

    @property
    def device(self):
        return self.lm_head.weight.device

    def new_cache(self, batch_size, max_length):
        """An empty KV cache of ``max_length`` positions for ``batch_size`` rows on the model's device."""
        c = self.config
        if type(batch_size) is not int or batch_size < 1:
            raise ValueError('batch_size must be a positive int')
        if type(max_length) is not int or not 1 <= max_length <= c.max_position_embeddings:
            raise ValueError(f'max_length must be an int in [1, {c.max_position_embeddings}]')
        if self.device.type != 'cuda':
            raise ValueError('the weights are not on a ROCm device (load or move them first)')
        shape = (batch_size, c.num_key_value_heads, max_length, c.head_dim)

        def layer_buffers():
            return [torch.empty(shape, device=self.device, dtype=torch.bfloat16) for _ in self.model.layers]
        return KVCache(layer_buffers(), layer_buffers(), max_length, batch_size, self._cache_owner)

    # ------------------------------------------------------------------ forward
    def _forward(self, input_ids, cache, logits_to_keep, *, validate_ids=True, start_dev=None):
        from transformers.modeling_outputs import CausalLMOutputWithPast
        if input_ids.ndim != 2 or input_ids.dtype not in (torch.int32, torch.int64) or \
                input_ids.device != self.device or not input_ids.is_contiguous():
            raise ValueError('Contiguous integer ROCm [B,S] input_ids on model device required')
        b, s = input_ids.shape
        if b < 1 or s < 1:
            raise ValueError('Nonempty batch/sequence required')
        cache.admit(self._cache_owner, b, s)
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
            layers = self.model.layers
            h = None  # the next layer's normed input when the previous down projection formed it
            for i, layer in enumerate(layers):
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
                if h is None:
                    h = kernels.rms_norm(x, layer.input_layernorm.weight, layer.input_layernorm.eps)
                q, k, v = _projections(h, [a.q_proj.weight, a.k_proj.weight, a.v_proj.weight], self.gemv)
                q = q.view(b, s, a.num_heads, d)
                k = k.view(b, s, a.num_kv_heads, d)
                v = v.view(b, s, a.num_kv_heads, d)
                if start_dev is None and a.q_norm.eps == a.k_norm.eps and _ops.norm_rope_qk_ok(q, k, d) and \
                        all(t.is_contiguous() for t in (q, k, v)):
                    # Q/K-norm + RoPE of both tensors and the K/V cache append in one launch
                    q = _ops.norm_rope_qk_cache_fwd(q, k, v, a.q_norm.weight, a.k_norm.weight, cos, sin,
                                                    cache.keys[i], cache.values[i], start, a.q_norm.eps)
                else:
                    q = kernels.norm_rope(q, a.q_norm.weight, cos, sin, a.q_norm.eps)
                    k = kernels.norm_rope(k, a.k_norm.weight, cos, sin, a.k_norm.eps)
                    kernels.append(k, v, cache.keys[i], cache.values[i], start, start_dev)
                y = kernels.attention(q, cache.keys[i], cache.values[i], start, split_decode=self.split_decode,
                                      start_dev=start_dev).reshape(b, s, -1)
                x = _residual_projection(x, y, a.o_proj.weight, self.gemv)
                h = kernels.rms_norm(x, layer.post_attention_layernorm.weight, layer.post_attention_layernorm.eps)
                m = layer.mlp
                if b * s <= 8 and self.gemv:
                    y = swiglu(kernels.linear(h, m.gate_proj.weight, gemv=True),
                               kernels.linear(h, m.up_proj.weight, gemv=True))
                else:
                    y = gate_up_swiglu(h, m.gate_proj.weight, m.up_proj.weight, optimized=True)
                if i + 1 < len(layers):  # the next layer's input norm rides with this residual sum
                    x, h = _residual_projection(x, y, m.down_proj.weight, self.gemv,
                                                layers[i + 1].input_layernorm)
                else:
                    x, h = _residual_projection(x, y, m.down_proj.weight, self.gemv), None
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


def _generation_config(config):
    """HF generation defaults (EOS / pad ids) derived from the model config, or None."""
    try:
        from transformers import GenerationConfig
        return GenerationConfig.from_model_config(config)
    except Exception:  # pragma: no cover - generation defaults only
        return None


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
    def reset(self):
        """Forget the request (cache contents, length, finished rows); memory and any captured step
        graph stay valid for the next prompt."""
        self.cache.reset()
        self.length.zero_()
        self.done.zero_()
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
    """A fixed-shape greedy request (prefill + ``max_new_tokens`` tokens, no early EOS) replayed from
    HIP graphs, with the call contract of ``inference/model.py:191-225``: the constructor captures,
    each call copies a prompt of the captured shape in and returns the [B, S + max_new_tokens]
    tokens.  Single-stream and non-reentrant; the returned tensor aliases request storage until
    the next call.

    Two graphs serve any token budget: one for the prefill (embedding through the first greedy
    token) and one decode step whose position-dependent kernels read the cache length from device
    memory, replayed ``max_new_tokens - 1`` times.  The graph size is therefore fixed (about 36
    layers x 8 kernels per graph for Qwen3-8B) whatever the budget.  Capturing the whole request as
    one graph instead would grow with prompt and budget (~157 K kernel nodes for a 2048-token prompt
    and 256 new tokens) and is not done.
    """

    @torch.inference_mode()
    def __init__(self, model, input_ids, *, max_new_tokens):
        if type(max_new_tokens) is not int or max_new_tokens < 1:
            raise ValueError('max_new_tokens must be a positive int (the fixed token budget)')
        if input_ids.ndim != 2 or input_ids.device != model.device or \
                input_ids.dtype not in (torch.int32, torch.int64) or min(input_ids.shape) < 1:
            raise ValueError('a nonempty integer [B, S] prompt on the model device is required')
        _check_vocab(model, input_ids)
        b, s = input_ids.shape
        self.model, self.shape, self.budget, self.busy = model, (b, s), max_new_tokens, False
        self.input = input_ids.clone()
        dev = model.device
        self.cache = model.new_cache(b, s + max_new_tokens)
        self.output = torch.zeros((b, s + max_new_tokens), device=dev, dtype=torch.int64)
        self.current = torch.zeros((b, 1), device=dev, dtype=torch.int64)
        self.length = torch.zeros((1,), device=dev, dtype=torch.int64)
        self.done = torch.zeros((b,), device=dev, dtype=torch.bool)
        stream = torch.cuda.Stream(device=dev)
        stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(stream):   # one eager pass: workspaces and kernels are warm before capture
            self._prefill()
            if max_new_tokens > 1:
                self._step()
        self.prefill_graph = torch.cuda.CUDAGraph()
        self.cache.reset()
        with torch.cuda.graph(self.prefill_graph, stream=stream):
            self._prefill()
        self.step_graph = None
        if max_new_tokens > 1:
            self.step_graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.step_graph, stream=stream):
                self._step()
        torch.cuda.current_stream(dev).wait_stream(stream)
        self.cache.reset()

    def _prefill(self):
        """Prompt -> cache, first greedy token at position S; device length := S."""
        b, s = self.shape
        self.cache.length = 0
        self.output[:, :s].copy_(self.input)
        logits = self.model._forward(self.input, self.cache, 1, validate_ids=False).logits[:, 0, :]
        self.done.zero_()
        kernels.select(logits, self.output, self.current, self.done, s, (), 0)
        self.length.zero_()
        kernels.advance(self.length, s)

    def _step(self):
        """One cached token at the device-resident length L: token L+1 is written; L += 1."""
        self.cache.length = self.shape[1]   # host-side bound checks only; positions come from self.length
        logits = self.model._forward(self.current, self.cache, 1, validate_ids=False,
                                     start_dev=self.length).logits[:, 0, :]
        kernels.select(logits, self.output, self.current, self.done, 1, (), 0, position_dev=self.length)
        kernels.advance(self.length, 1)

    @torch.inference_mode()
    def __call__(self, input_ids):
        if self.busy:
            raise RuntimeError('a CapturedGreedyRequest serves one call at a time')
        if tuple(input_ids.shape) != self.shape or input_ids.device != self.model.device or \
                input_ids.dtype != self.input.dtype:
            raise ValueError(f'prompt must match the captured {self.shape} {self.input.dtype} on {self.model.device}')
        self.busy = True
        try:
            _check_vocab(self.model, input_ids)
            self.input.copy_(input_ids)
            self.prefill_graph.replay()
            for _ in range(self.budget - 1):
                self.step_graph.replay()
            return self.output
        finally:
            self.busy = False


def _check_vocab(model, ids):
    if not bool(((ids >= 0) & (ids < model.config.vocab_size)).all()):
        raise ValueError('token id outside the vocabulary')
