"""The C ABI: libq3hip.so loads on a GPU-less host and exports exactly what include/q3hip.h declares.

No compute is launched here; argument rejection (Q3_ERR_INVALID) is checked because it happens on
the host before any launch.
"""
import ctypes
import os
import re

from conftest import ROOT

from qwen3_triton import _hip as H

HEADER = os.path.join(ROOT, "include", "q3hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(q3_\w+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(H.LIB_PATH)
    names = declared()
    assert len(names) >= 20
    for n in sorted(names):
        assert hasattr(lib, n), n


def test_python_signatures_cover_the_header_exactly():
    assert declared() == set(H.SIGNATURES)


def test_version_and_error_strings():
    lib = H.load()
    assert lib.q3_abi_version() >= 1
    assert b"invalid argument" in lib.q3_error_string(100000)
    assert lib.q3_error_string(0) == b"success"


def test_invalid_arguments_are_rejected_before_launch():
    lib = H.load()
    # null pointers / zero sizes / unsupported dtype never reach a launch
    assert lib.q3_rmsnorm_fwd(2, None, None, None, 4, 128, 1e-6, None) == 100000
    assert lib.q3_swiglu_fwd(7, 1, 1, 1, 16, None) == 100000
    assert lib.q3_gemm_nt(0, 0, 16, 8, 16, 8, 16, 8, 1, 1, 8, 1.0, 0, None) == 100000  # fp32 in: not MFMA
    assert lib.q3_gemm_nt(2, 0, 16, 8, 16, 8, 16, 8, 1, 1, 12, 1.0, 0, None) == 100000  # K % 8 != 0


def test_noalloc_decode_attention_rejects_oversize_before_any_gpu_call():
    """The no-allocation decode attention refuses a request whose split partials exceed its fixed
    scratch array (Q3_ERR_SCRATCH) before touching the device or any pointer."""
    lib = H.load()
    assert b"scratch" in lib.q3_error_string(100001)
    limit = 16 << 20
    # 128-key splits: B 8 x Hq 32 fits 126 splits
    assert H.query("q3_decode_attention_workspace_bytes", 8, 32, 8, 16128) <= limit
    assert H.query("q3_decode_attention_workspace_bytes", 8, 32, 8, 16129) > limit
    args = [2, None, 0, 0, None, None, 0, 0, None, None, 1e-6, None, None, 0, None, None, 0, 0, None, 0, 0,
            8, 32, 8, 16256, None, 16256, 128, 0.088, None]
    assert lib.q3_decode_step_attention_noalloc(*args) == 100001
