"""``ops/triton/rms_norm.py:118-138`` (``rms_norm_triton``) on the HIP RMSNorm kernels."""
import torch

from qwen3_triton.kernels import _ops


def _validate(x, weight):
    if not x.is_cuda or not weight.is_cuda:
        raise ValueError("rms_norm_triton requires ROCm tensors")
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"unsupported input dtype: {x.dtype}")
    if weight.dtype != x.dtype:
        raise TypeError("x and weight must have the same dtype")
    if x.shape[-1] != weight.numel():
        raise ValueError("weight length must equal x.shape[-1]")
    if x.shape[-1] > 65536:
        raise ValueError("hidden dimension is too large for this first kernel")


class _RMSNormFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, eps):
        _validate(x, weight)
        x = x.contiguous()
        w = weight.contiguous().view(-1)
        ctx.save_for_backward(x, w)
        ctx.eps = eps
        ctx.wshape = weight.shape
        return _ops.rmsnorm_fwd(x, w, eps)

    @staticmethod
    def backward(ctx, grad_output):
        x, w = ctx.saved_tensors
        dx, dw = _ops.rmsnorm_bwd(x, w, grad_output.contiguous(), ctx.eps)
        return dx, dw.view(ctx.wshape), None


def rms_norm_triton(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Apply Qwen RMSNorm (HIP forward and backward)."""
    return _RMSNormFunction.apply(x, weight, eps)
