"""Host-side validation of the reference-shaped wrappers (no GPU needed: it fails before launch)."""
import pytest
import torch

from qwen3_triton.kernels.norm import rms_norm
from qwen3_triton.kernels.linear import matmul
from qwen3_triton.kernels.activation import swiglu
from qwen3_triton.kernels.rotary import apply_rotary
from ops.triton.rms_norm import rms_norm_triton
from ops.triton.silu_and_mul import silu_and_mul_triton


def test_cpu_tensors_are_rejected_no_fallback():
    x = torch.randn(2, 8)
    with pytest.raises(ValueError):
        rms_norm(x, torch.ones(8))
    with pytest.raises(ValueError):
        matmul(x, x.t())
    with pytest.raises(ValueError):
        swiglu(x, x)
    with pytest.raises(ValueError):
        rms_norm_triton(x, torch.ones(8))
    with pytest.raises(ValueError):
        silu_and_mul_triton(x, x)
    with pytest.raises(ValueError):
        apply_rotary(torch.randn(1, 2, 3, 4), torch.randn(1, 2, 4), torch.randn(1, 2, 4))
