"""Single-GPU prefill, cached decode and greedy Qwen3 generation on HIP kernels."""
from .model import CapturedGreedyRequest, DecodeSession, KVCache, TritonQwen3Inference

__all__ = ['KVCache', 'TritonQwen3Inference', 'CapturedGreedyRequest', 'DecodeSession']
