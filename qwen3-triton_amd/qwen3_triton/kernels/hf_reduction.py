"""``qwen3_triton/kernels/hf_reduction.py``: the gate for replaying one PyTorch CUDA build's row-mean
summation order.  The reference enables it only for that CUDA build (``hf_reduction.py:12,15-19``: on a
ROCm build the gate is closed); here it is closed on every input, and the RMSNorm kernels sum in
their own fixed order."""


def supports_hf_reduction(x):
    """``hf_reduction.py:15-19``: whether the replayed summation order applies to ``x``."""
    return False
