"""``ops/triton/fused_qk_norm_rope.py:237-273``: fused Q/K RMSNorm + RoPE, q/k [B,S,H,D]."""

from qwen3_triton.kernels.norm_rope import norm_rope_pair


def _check(x, w, cos, sin):
    if not x.is_cuda:
        raise ValueError("fused_qk_norm_rope requires ROCm tensors")
    if x.ndim != 4 or w.numel() != x.shape[-1] or cos.shape != (x.shape[0], x.shape[1], x.shape[3]) or \
            sin.shape != cos.shape or x.shape[-1] % 2:
        raise ValueError("expected x=[B,S,H,D], weight=[D], cos/sin=[B,S,D] with even D")
    if w.dtype != x.dtype or cos.dtype != x.dtype or sin.dtype != x.dtype:
        raise TypeError("weight and cos/sin must have the dtype of x")


def fused_qk_norm_rope_triton(q, k, q_weight, k_weight, cos, sin, eps=1e-6):
    """Fused Q/K RMSNorm + RoPE: one HIP launch for both tensors per direction (one per tensor for
    shapes outside the vector path)."""
    for x, w in ((q, q_weight), (k, k_weight)):
        _check(x, w, cos, sin)
    return norm_rope_pair(q, k, q_weight, k_weight, cos, sin, eps)
