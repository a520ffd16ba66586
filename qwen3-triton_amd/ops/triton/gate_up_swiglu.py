"""``ops/triton/gate_up_swiglu.py:178-288`` (``gate_up_swiglu_triton``)."""
from qwen3_triton.kernels.mlp_precision import gate_up_swiglu


def gate_up_swiglu_triton(x, gate_weight, up_weight):
    """silu(X Wg^T) * (X Wu^T) with the HIP GEMM + SwiGLU kernels, trainable."""
    return gate_up_swiglu(x, gate_weight, up_weight)
