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


def test_reference_api_modules_and_defaults():
    """Names the reference exports on this path exist with its defaults."""
    import inspect
    from qwen3_triton.kernels import mlp, attention_precision
    from qwen3_triton.inference import kernels as ik
    assert callable(mlp.gate_up_swiglu) and callable(ik.sliced_linear) and callable(ik.tiled_prefill_gate_up)
    sig = inspect.signature(attention_precision.candidate).parameters
    assert {k: sig[k].default for k in ("lse_fma", "native_delta", "native_dq", "sum_fma", "xor_sum")} == \
        dict(lse_fma=False, native_delta=False, native_dq=False, sum_fma=False, xor_sum=True)
    assert attention_precision.f32(0.1) == 0.10000000149011612
    assert attention_precision.f32(128 ** -0.5) != 128 ** -0.5
    # the reference-order replay modules: importable, and their gates closed (callers keep their route)
    from qwen3_triton.inference import accumulation
    from qwen3_triton.kernels import hf_reduction
    assert accumulation.strategy(1, 4096, 4096) is None
    assert accumulation.linear(torch.zeros(1, 8), torch.zeros(8, 8)) is None
    assert accumulation.short_norm(torch.zeros(1, 4096), torch.zeros(4096), 1e-6) is None
    assert hf_reduction.supports_hf_reduction(torch.zeros(16, 128)) is False


def test_unknown_variant_message():
    """``configuration.py:21``: an unknown preset name raises with the reference's message."""
    import pytest
    from qwen3_triton.configuration import options_for_variant
    with pytest.raises(ValueError, match='Unknown Triton variant: nope'):
        options_for_variant('nope')


def test_precision_model_option_validation():
    from qwen3_triton.model import _optimization_options, _precision_items
    from qwen3_triton.configuration import OptimizationOptions
    import pytest
    assert dict(_precision_items(None)) == dict(xor_sum=True, lse_fma=True, native_delta=True, native_dq=True,
                                                sum_fma=True)
    with pytest.raises(ValueError, match='Explicit five boolean precision options required'):
        _precision_items(dict(xor_sum=True))
    with pytest.raises(ValueError):
        _precision_items(dict(xor_sum=1, lse_fma=True, native_delta=True, native_dq=True, sum_fma=True))
    o = _optimization_options(None)
    assert isinstance(o, OptimizationOptions) and not o.mlp_fusion and not o.linear_optimized
    # the caller's order is kept (the reference stores ``tuple(precision_options.items())``)
    order = dict(sum_fma=False, xor_sum=True, native_dq=True, lse_fma=False, native_delta=True)
    assert _precision_items(order) == tuple(order.items())

    class Foreign:        # attributes are taken as given, not coerced to bool
        mlp_fusion = 1
    assert _optimization_options(Foreign()).mlp_fusion == 1


def test_architecture_rules():
    import pytest
    from transformers import Qwen3Config
    from qwen3_triton._checkpoint import check_architecture
    check_architecture(Qwen3Config(head_dim=128))
    for kw, what in [(dict(hidden_act="gelu"), "SiLU"), (dict(attention_bias=True), "bias"),
                     (dict(num_attention_heads=6, num_key_value_heads=4), "GQA"),
                     (dict(rope_scaling={"rope_type": "linear", "factor": 2.0}), "RoPE")]:
        with pytest.raises(ValueError, match=what):
            check_architecture(Qwen3Config(head_dim=128, **kw))


def test_captured_request_rejects_bad_budgets_before_any_gpu_work():
    import pytest
    from qwen3_triton.inference import CapturedGreedyRequest
    for budget in (0, -1, 2.0):
        with pytest.raises(ValueError):
            CapturedGreedyRequest(object(), None, max_new_tokens=budget)
