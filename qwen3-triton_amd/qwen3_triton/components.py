"""Training components (the reference's "precision" path), ``qwen3_triton/components.py:1-54``.

``HFOrderNorm`` / ``Attention`` / ``MLP`` / ``DecoderLayer`` / ``Backbone`` keep the reference's
module structure and option switches (the q/k/v projections keep their own parameters and run
through one shared-input projection op whose backward is a single dX GEMM): ``norm_rope_fusion`` selects the fused per-head RMSNorm +
RoPE kernel, ``mlp_fusion`` the fused gate/up + SwiGLU + down block (``mlp_block``: SwiGLU backward in
the down projection's input-gradient GEMM epilogue).  The decoder layer hands each block its
residual input, so the residual sums ride in the epilogues of the o_proj and down_proj GEMMs.  The
reference's SM86 rounding-order options (``precision_options``) are accepted and select nothing on
gfx950.
"""
import torch

from ._model import TritonAttention, TritonDecoderLayer, TritonMLP, TritonNorm, TritonQwen3Model
from .kernels.activation import swiglu
from .kernels.attention import causal_attention_bshd
from .kernels.linear import linear_residual, shared_input_projections
from .kernels.math_precision import norm_rope, rms_norm
from .kernels.mlp_precision import mlp_block
from .kernels.norm import rms_norm_fork
from .kernels.norm_rope import norm_rope_pair
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

    def forward(self, x, positions, residual=None):
        b, s, _ = x.shape
        d = self.head_dim
        cos, sin = positions
        q, k, v = shared_input_projections(x, [self.q_proj.weight, self.k_proj.weight, self.v_proj.weight],
                                           optimized=self.q_proj.options.linear_optimized)
        q = q.view(b, s, self.num_heads, d)
        k = k.view(b, s, self.num_kv_heads, d)
        v = v.view(b, s, self.num_kv_heads, d)
        if getattr(self.options, 'norm_rope_fusion', False) and self.q_norm.eps == self.k_norm.eps:
            q, k = norm_rope_pair(q, k, self.q_norm.weight, self.k_norm.weight, cos, sin, self.q_norm.eps)
        elif getattr(self.options, 'norm_rope_fusion', False):
            q = norm_rope(q, self.q_norm.weight, cos, sin, self.q_norm.eps)
            k = norm_rope(k, self.k_norm.weight, cos, sin, self.k_norm.eps)
        else:
            q = apply_rotary(self.q_norm(q), cos, sin)
            k = apply_rotary(self.k_norm(k), cos, sin)
        y = causal_attention_bshd(q, k, v, scale=d ** -0.5).reshape(b, s, self.num_heads * d)
        if residual is None:
            return self.o_proj(y)
        return linear_residual(y, self.o_proj.weight, residual, optimized=self.o_proj.options.linear_optimized)


class MLP(TritonMLP):
    def forward(self, x, residual=None):
        opts = self.gate_proj.options
        if getattr(opts, 'mlp_fusion', False):
            return mlp_block(x, self.gate_proj.weight, self.up_proj.weight, self.down_proj.weight,
                             optimized=opts.linear_optimized, residual=residual)
        y = swiglu(self.gate_proj(x), self.up_proj(x))
        if residual is None:
            return self.down_proj(y)
        return linear_residual(y, self.down_proj.weight, residual, optimized=opts.linear_optimized)


class DecoderLayer(TritonDecoderLayer):
    def __init__(self, c, options):
        torch.nn.Module.__init__(self)
        self.self_attn = Attention(c, options)
        self.mlp = MLP(c, options)
        self.input_layernorm = HFOrderNorm(c.hidden_size, c.rms_norm_eps)
        self.post_attention_layernorm = HFOrderNorm(c.hidden_size, c.rms_norm_eps)

    def forward(self, x, position_embeddings):
        # ``_model.py:60-108`` layer order; x forks into the norm and the residual sum (one autograd node
        # whose backward adds both gradients), and each block adds its residual in its last GEMM.
        x, h = rms_norm_fork(x, self.input_layernorm.weight, self.input_layernorm.eps)
        x = self.self_attn(h, position_embeddings, residual=x)
        x, h = rms_norm_fork(x, self.post_attention_layernorm.weight, self.post_attention_layernorm.eps)
        return self.mlp(h, residual=x)


class Backbone(TritonQwen3Model):
    decoder_class = DecoderLayer

    def __init__(self, c, options):
        super().__init__(c, options)
        self.norm = HFOrderNorm(c.hidden_size, c.rms_norm_eps)
