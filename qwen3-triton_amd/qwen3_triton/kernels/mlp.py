"""``qwen3_triton/kernels/mlp.py:34-56`` (``gate_up_swiglu``): the gate and up projections and SwiGLU
as one trainable op.  The reference keeps this module beside ``mlp_precision``.  Both run the same
HIP path here.  The forward is one dual-weight matrix-core GEMM that stores G, U and
Y = silu(G) * U.  The backward is the SwiGLU backward plus packed dX / dW GEMMs."""
from .mlp_precision import _GateUp


def gate_up_swiglu(x, gate_weight, up_weight, *, optimized=False):
    return _GateUp.apply(x, gate_weight, up_weight, optimized)
