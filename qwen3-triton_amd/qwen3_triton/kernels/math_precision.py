"""Names of ``qwen3_triton/kernels/math_precision.py:23-96`` on the HIP kernels.

The reference replays PyTorch-CUDA reduction orders here (an SM86/CUDA-only bit-parity target,
``kernels/hf_reduction.py:12-18``).  This build computes in fp32 with a single final rounding;
the ``fma`` switch of ``swiglu`` is accepted and has no effect.
"""
from .activation import swiglu as _swiglu
from .norm import rms_norm as _rms_norm
from .norm_rope import norm_rope as _norm_rope


def rms_norm(x, w, eps=1e-6):
    return _rms_norm(x, w, eps)


def norm_rope(x, w, cos, sin, eps=1e-6):
    return _norm_rope(x, w, cos, sin, eps)


def swiglu(g, u, *, fma=True):
    return _swiglu(g, u)
