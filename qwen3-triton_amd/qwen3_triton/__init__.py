"""Qwen3 decoder operator set on MI355X (gfx950) HIP kernels.

Keeps the module and ``autograd.Function`` API of the reference package ``qwen3_triton``
(wuyii8941/qwen3-triton): ``qwen3_triton.kernels.*``, ``qwen3_triton.components``,
``qwen3_triton.inference``.  The model classes are imported lazily so that the operator modules do
not pull in ``transformers``.
"""
__all__ = ["TritonQwen3ForCausalLM", "PrecisionQwen3ForCausalLM", "model_for_variant"]


def __getattr__(name):
    if name in __all__:
        from . import model
        if name == "TritonQwen3ForCausalLM":
            return model.PrecisionQwen3ForCausalLM
        return getattr(model, name)
    raise AttributeError(name)
