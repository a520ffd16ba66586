"""``ops/triton/silu_and_mul.py:79-121`` (``silu_and_mul_triton``) on the HIP SwiGLU kernels."""
import torch

from qwen3_triton.kernels import _ops


class _SiluAndMul(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gate, up):
        ctx.save_for_backward(gate, up)
        return _ops.swiglu_fwd(gate, up)

    @staticmethod
    def backward(ctx, grad_output):
        gate, up = ctx.saved_tensors
        return _ops.swiglu_bwd(gate, up, grad_output.contiguous())


def silu_and_mul_triton(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """SwiGLU activation silu(gate) * up."""
    if not (gate.is_cuda and up.is_cuda):
        raise ValueError("silu_and_mul_triton requires ROCm tensors")
    if gate.shape != up.shape:
        raise ValueError("gate and up must have the same shape")
    if not (gate.is_floating_point() and up.is_floating_point()):
        raise TypeError("gate and up must be floating-point tensors")
    if gate.dtype != up.dtype:
        raise TypeError("gate and up must have the same dtype")
    return _SiluAndMul.apply(gate.contiguous(), up.contiguous())
