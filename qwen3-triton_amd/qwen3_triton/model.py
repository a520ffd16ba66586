"""Public Qwen3 training model and variant factory (``qwen3_triton/model.py:1-23``)."""
from dataclasses import fields, replace

from ._model import TritonQwen3ForCausalLM
from .components import Backbone, HFOrderNorm  # noqa: F401
from .configuration import OptimizationOptions, options_for_variant


class PrecisionQwen3ForCausalLM(TritonQwen3ForCausalLM):
    backbone_class = Backbone

    def __init__(self, config, options=None, *, precision_options=None, require_8b_shape=True):
        if precision_options is None:
            precision_options = dict(xor_sum=True, lse_fma=True, native_delta=True, native_dq=True, sum_fma=True)
        if set(precision_options) != {'xor_sum', 'lse_fma', 'native_delta', 'native_dq', 'sum_fma'} or \
                any(type(v) is not bool for v in precision_options.values()):
            raise ValueError('Explicit five boolean precision options required')
        if require_8b_shape and not (config.num_hidden_layers == 36 and config.hidden_size == 4096 and
                                     config.head_dim == 128):
            raise ValueError('The precision model is qualified for the Qwen3-8B shape only')
        if options is None:
            options = OptimizationOptions(**{f.name: False for f in fields(OptimizationOptions)
                                             if f.name != 'precision_options'})
        elif not isinstance(options, OptimizationOptions):
            options = OptimizationOptions(**{f.name: getattr(options, f.name, False)
                                             for f in fields(OptimizationOptions) if f.name != 'precision_options'})
        options = replace(options, precision_options=tuple(precision_options.items()))
        super().__init__(config, options)


def model_for_variant(config, name, *, precision_options=None):
    return PrecisionQwen3ForCausalLM(config, options_for_variant(name), precision_options=precision_options)
