"""Training components (the reference's "precision" path), ``qwen3_triton/components.py:1-54``.

``HFOrderNorm`` / ``Attention`` / ``MLP`` / ``DecoderLayer`` / ``Backbone`` keep the reference's
module structure and option switches (the q/k/v projections keep their own parameters and run
through one shared-input projection op whose backward is a single dX GEMM): ``norm_rope_fusion`` selects the fused per-head RMSNorm +
RoPE kernel, ``mlp_fusion`` the fused gate/up + SwiGLU + down block (``mlp_block``: SwiGLU backward in
the down projection's input-gradient GEMM epilogue).  The reference's SM86 rounding-order options
(``precision_options``) are accepted and select nothing on gfx950.
"""
import torch

from ._model import TritonAttention, TritonDecoderLayer, TritonMLP, TritonNorm, TritonQwen3Model
from .kernels.activation import swiglu
from .kernels.attention import causal_attention_bshd
from .kernels.linear import shared_input_projections
from .kernels.math_precision import norm_rope, rms_norm
from .kernels.mlp_precision import mlp_block
from .kernels.rotary import apply_rotary


class HFOrderNorm(TritonNorm):
    def forward(self, x):
        return rms_norm(x, self.weight, self.eps)


class Attention(TritonAttention):
    def __init__(self, config, options):
        super().__init__(config, options)
        self.precision_options = dict(getattr(options, 'precision_options', ()))
        self.q_norm = HFOrderNorm(self.head_dim, config.rms_norm_eps)
        self.k_norm = HFOrderNorm(self.head_dim, config.rms_norm_eps)

    def forward(self, x, positions):
        b, s, _ = x.shape
        d = self.head_dim
        cos, sin = positions
        q, k, v = shared_input_projections(x, [self.q_proj.weight, self.k_proj.weight, self.v_proj.weight],
                                           optimized=self.q_proj.options.linear_optimized)
        q = q.view(b, s, self.num_heads, d)
        k = k.view(b, s, self.num_kv_heads, d)
        v = v.view(b, s, self.num_kv_heads, d)
        if getattr(self.options, 'norm_rope_fusion', False):
            q = norm_rope(q, self.q_norm.weight, cos, sin, self.q_norm.eps)
            k = norm_rope(k, self.k_norm.weight, cos, sin, self.k_norm.eps)
        else:
            q = apply_rotary(self.q_norm(q), cos, sin)
            k = apply_rotary(self.k_norm(k), cos, sin)
        y = causal_attention_bshd(q, k, v, scale=d ** -0.5)
        return self.o_proj(y.reshape(b, s, self.num_heads * d))


class MLP(TritonMLP):
    def forward(self, x):
        opts = self.gate_proj.options
        if getattr(opts, 'mlp_fusion', False):
            return mlp_block(x, self.gate_proj.weight, self.up_proj.weight, self.down_proj.weight,
                             optimized=opts.linear_optimized)
        else:
            y = swiglu(self.gate_proj(x), self.up_proj(x))
        return self.down_proj(y)


class DecoderLayer(TritonDecoderLayer):
    def __init__(self, c, options):
        torch.nn.Module.__init__(self)
        self.self_attn = Attention(c, options)
        self.mlp = MLP(c, options)
        self.input_layernorm = HFOrderNorm(c.hidden_size, c.rms_norm_eps)
        self.post_attention_layernorm = HFOrderNorm(c.hidden_size, c.rms_norm_eps)


class Backbone(TritonQwen3Model):
    decoder_class = DecoderLayer

    def __init__(self, c, options):
        super().__init__(c, options)
        self.norm = HFOrderNorm(c.hidden_size, c.rms_norm_eps)
