"""Standalone operator API with the call signatures of the reference's ``ops.triton`` package.

The implementations are hand-written HIP kernels for gfx950 (``qwen3_triton/libq3hip.so``); the
package name is kept so that callers of ``ops.triton.*`` work unchanged.
"""
