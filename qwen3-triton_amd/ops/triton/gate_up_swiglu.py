"""``ops/triton/gate_up_swiglu.py:178-288`` (``gate_up_swiglu_triton``)."""
from qwen3_triton.kernels.mlp_precision import gate_up_swiglu


def gate_up_swiglu_triton(x, gate_weight, up_weight):
    """silu(X Wg^T) * (X Wu^T) with the HIP GEMM + SwiGLU kernels, trainable.  The argument checks are
    the reference's (``gate_up_swiglu.py:278-287``); strided operands are taken as it takes them
    (contiguous copies)."""
    if not all(t.is_cuda for t in (x, gate_weight, up_weight)):
        raise ValueError("gate_up_swiglu_triton requires ROCm tensors")
    if x.ndim < 2 or gate_weight.ndim != 2 or up_weight.shape != gate_weight.shape:
        raise ValueError("expected x [..., K] and matching weights [N, K]")
    if x.shape[-1] != gate_weight.shape[1]:
        raise ValueError("x and weight K dimensions must match")
    if not (x.is_floating_point() and gate_weight.is_floating_point() and up_weight.is_floating_point()):
        raise TypeError("all inputs must be floating-point tensors")
    if not (x.dtype == gate_weight.dtype == up_weight.dtype):
        raise TypeError("all inputs must have the same dtype")
    return gate_up_swiglu(x.contiguous(), gate_weight.contiguous(), up_weight.contiguous())
