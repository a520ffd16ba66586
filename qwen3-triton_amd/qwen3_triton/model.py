"""Public Qwen3 training model and variant factory (``qwen3_triton/model.py:1-23``).

``PrecisionQwen3ForCausalLM`` is the training model on the ``components`` modules.  It carries
the reference's five precision switches as a tuple inside the options.  On gfx950 every kernel
computes in fp32 and rounds once, so the switches are validated and recorded but select nothing.
"""
from dataclasses import fields, replace

from ._model import TritonQwen3ForCausalLM
from .components import Backbone, HFOrderNorm  # noqa: F401
from .configuration import OptimizationOptions, options_for_variant

PRECISION_SWITCHES = ('xor_sum', 'lse_fma', 'native_delta', 'native_dq', 'sum_fma')


def _precision_items(precision_options):
    """The five switches as a tuple of (name, bool) in the caller's order; all on when none are given."""
    if precision_options is None:
        return tuple((name, True) for name in PRECISION_SWITCHES)
    given = dict(precision_options)
    if sorted(given) != sorted(PRECISION_SWITCHES) or not all(type(v) is bool for v in given.values()):
        raise ValueError('Explicit five boolean precision options required')
    return tuple(given.items())


def _optimization_options(options):
    """``OptimizationOptions`` from None (every switch off), an ``OptimizationOptions``, or any object
    whose like-named attributes are taken as they are (missing ones off)."""
    if isinstance(options, OptimizationOptions):
        return options
    switches = [f.name for f in fields(OptimizationOptions) if f.name != 'precision_options']
    return OptimizationOptions(**{name: getattr(options, name, False) for name in switches})


def _is_8b_shape(config):
    return (config.num_hidden_layers, config.hidden_size, config.head_dim) == (36, 4096, 128)


class PrecisionQwen3ForCausalLM(TritonQwen3ForCausalLM):
    backbone_class = Backbone

    def __init__(self, config, options=None, *, precision_options=None, require_8b_shape=True):
        switches = _precision_items(precision_options)
        if require_8b_shape and not _is_8b_shape(config):
            raise ValueError('the precision model is qualified for the Qwen3-8B shape (36 layers, hidden 4096, '
                             'head_dim 128); pass require_8b_shape=False for other shapes')
        super().__init__(config, replace(_optimization_options(options), precision_options=switches))


def model_for_variant(config, name, *, precision_options=None):
    return PrecisionQwen3ForCausalLM(config, options_for_variant(name), precision_options=precision_options)
