"""HIP-backed operator modules named after the reference's ``qwen3_triton/kernels/*``."""
