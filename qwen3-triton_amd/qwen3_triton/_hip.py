"""Loader and call shim for libq3hip.so (the C ABI declared in include/q3hip.h).

PyTorch supplies device memory and the current HIP stream; every numerical operation runs in a
hand-written gfx950 kernel behind this ABI.  There is no fallback: if the library is missing, or
a tensor is not on a ROCm device, the call raises.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libq3hip.so")

F32, F16, BF16 = 0, 1, 2
_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/q3hip.h one-to-one.
SIGNATURES: dict[str, tuple] = {
    "q3_error_string": (ctypes.c_char_p, [_i32]),
    "q3_abi_version": (_i32, []),
    "q3_rmsnorm_fwd": (_i32, [_i32, _p, _p, _p, _i64, _i64, _f32, _p]),
    "q3_rmsnorm_bwd_workspace_bytes": (_sz, [_i64, _i64]),
    "q3_rmsnorm_bwd": (_i32, [_i32, _p, _p, _p, _p, _p, _p, _i64, _i64, _f32, _p]),
    "q3_rmsnorm_bwd_add": (_i32, [_i32, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _f32, _p]),
    "q3_norm_rope_fwd": (_i32, [_i32, _p, _p, _p, _p, _p, _i64, _i64, _i64, _f32, _p]),
    "q3_norm_rope_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "q3_norm_rope_bwd": (_i32, [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _f32, _p]),
    "q3_norm_rope_qk_fwd": (_i32, [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _p]),
    "q3_norm_rope_qk_cache_fwd": (_i32, [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                         _i64, _i64, _f32, _p]),
    "q3_norm_rope_qk_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "q3_norm_rope_qk_bwd": (_i32, [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64,
                                    _f32, _p]),
    "q3_rope_tables": (_i32, [_i32, _p, _i32, _p, _p, _p, _i64, _i64, _p]),
    "q3_rope_apply": (_i32, [_i32, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _i32, _p]),
    "q3_swiglu_fwd": (_i32, [_i32, _p, _p, _p, _i64, _p]),
    "q3_swiglu_bwd": (_i32, [_i32, _p, _p, _p, _p, _p, _i64, _p]),
    "q3_swiglu_bwd_2d": (_i32, [_i32, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _p]),
    "q3_copy2d": (_i32, [_i32, _p, _i64, _p, _i64, _i64, _i64, _p]),
    "q3_transpose2d": (_i32, [_i32, _p, _i64, _p, _i64, _i64, _i64, _p]),
    "q3_add": (_i32, [_i32, _p, _p, _p, _i64, _p]),
    "q3_cast": (_i32, [_i32, _i32, _p, _p, _i64, _p]),
    "q3_fill": (_i32, [_i32, _p, _f32, _i64, _p]),
    "q3_positions": (_i32, [_p, _i64, _i64, _i64, _p, _p]),
    "q3_transpose": (_i32, [_i32, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "q3_embedding_fwd": (_i32, [_i32, _p, _i32, _p, _p, _p, _i64, _i64, _i64, _p]),
    "q3_embedding_bwd_workspace_bytes": (_sz, [_i64]),
    "q3_embedding_bwd": (_i32, [_i32, _p, _i32, _p, _p, _p, _i64, _i64, _i64, _p]),
    "q3_gemm_nt": (_i32, [_i32, _i32, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _f32, _i32, _p]),
    "q3_gemm_gate_up_swiglu": (_i32, [_i32, _p, _i64, _p, _p, _i64, _p, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "q3_gemm_gate_up_swiglu_t": (_i32, [_i32, _p, _i64, _p, _p, _i64, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _i64,
                                        _p]),
    "q3_gemm_nt_residual": (_i32, [_i32, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _p]),
    "q3_gemm_nt_residual_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "q3_gemm_nt_residual_ws": (_i32, [_i32, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _p, _sz, _p]),
    "q3_gemm_nt_residual_norm_ws": (_i32, [_i32, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _f32, _p, _i64, _i64,
                                            _i64, _i64, _p, _sz, _p]),
    "q3_gemm_swiglu_bwd": (_i32, [_i32, _p, _i64, _p, _i64, _p, _p, _i64, _p, _p, _i64, _p, _p, _i64, _i64, _i64,
                                  _i64, _p]),
    "q3_gemm_nt_multi": (_i32, [_i32, _p, _i64, _i32, _p, _i64, _p, _p, _p, _i64, _i64, _p]),
    "q3_attention_mfma_supported": (_i32, [_i32, _i64]),
    "q3_attention_seq_major": (_i32, [_i32, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _p]),
    "q3_attention_fwd": (_i32, [_i32, _p, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _i64, _p, _p, _i64, _i64,
                                 _i64, _i64, _i64, _i64, _f32, _p]),
    "q3_attention_bwd": (_i32, [_i32, _p, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _p, _i64,
                                 _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _p]),
    "q3_ce_shift_labels": (_i32, [_p, _p, _i64, _i64, _i64, _p]),
    "q3_ce_chunk_stats": (_i32, [_i32, _p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _p]),
    "q3_ce_finish": (_i32, [_p, _p, _i32, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "q3_ce_chunk_grad": (_i32, [_i32, _i32, _p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "q3_gemm_nt_ce_grad": (_i32, [_i32, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p,
                                  _p, _i64, _i64, _p]),
    "q3_gemm_nt_ce_stats": (_i32, [_i32, _p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _i64,
                                   _p]),
    "q3_gemm_nt_ce_stats_store": (_i32, [_i32, _p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _i64,
                                         _i64, _p, _i64, _p]),
    "q3_ce_chunk_grad_t": (_i32, [_i32, _p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _i64,
                                  _p]),
    "q3_gemv": (_i32, [_i32, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "q3_decode_linear": (_i32, [_i32, _p, _i64, _i64, _i64, _p, _f32, _i32, _i32, _p, _p, _p, _p, _p, _i64, _p]),
    "q3_kv_append": (_i32, [_i32, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p]),
    "q3_decode_attention_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "q3_decode_attention": (_i32, [_i32, _p, _i64, _i64, _p, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64,
                                    _i64, _p, _i64, _i64, _f32, _p]),
    "q3_decode_step_attention": (_i32, [_i32, _p, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _f32, _p, _p, _i64, _p, _p,
                                        _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _f32,
                                        _p]),
    "q3_decode_step_attention_noalloc": (_i32, [_i32, _p, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _f32, _p, _p, _i64,
                                                _p, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64,
                                                _i64, _f32, _p]),
    "q3_greedy_select_workspace_bytes": (_sz, [_i64]),
    "q3_greedy_select": (_i32, [_i32, _p, _i64, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _p, _p, _i32, _i64, _p]),
    "q3_advance": (_i32, [_p, _i64, _p]),
    "q3_gemm_strided": (_i32, [_i32, _i32, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _f32, _i32,
                                _p]),
}

_lib = None


def load():
    """Load libq3hip.so once and bind every symbol of SIGNATURES (raises if anything is absent)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libq3hip.so not built ({LIB_PATH}); run __graft_entry__.build()  -- no fallback")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Invoke a q3_* launcher; a non-zero status becomes RuntimeError."""
    rc = getattr(load(), name)(*args)
    if rc != 0:
        msg = load().q3_error_string(rc).decode()
        raise RuntimeError(f"{name} failed: {msg} (code {rc})")


def query(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))


def stream() -> int:
    """Handle of the current HIP stream of the current device (autograd may run on another thread,
    so it is read at call time)."""
    return torch.cuda.current_stream().cuda_stream


def code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; float32/float16/bfloat16 required") from None


def ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def require_device(*tensors: torch.Tensor) -> None:
    """The reference's same-device CUDA check (e.g. ``kernels/linear.py:47-48``); no CPU fallback."""
    dev = tensors[0].device
    for t in tensors:
        if not t.is_cuda:
            raise ValueError("ROCm device tensors required; no fallback")
        if t.device != dev:
            raise ValueError("all tensors must be on the same device")


def workspace(nbytes: int, device) -> torch.Tensor:
    """Caller-owned scratch for a kernel (the library never allocates)."""
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)
