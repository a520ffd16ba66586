"""``qwen3_triton/kernels/attention_precision.py:145-182`` (``f32``, ``candidate``).

The reference's ``candidate`` flags choose among SM86 rounding and reduction orders: exp2 or exp,
reverse tile order, 4-lane sums, a reciprocal PTX instruction, split dQ.  On gfx950 the flash
kernels have a single schedule: base-2 online softmax, fp32 accumulation and a deterministic GQA
reduction.  The flags keep the reference's names and defaults so calls stay valid.  They are
type-checked and do not change the result.
"""
import ctypes

from .attention import causal_attention


def f32(value):
    """``value`` rounded to the nearest fp32 number, returned as a Python float."""
    return ctypes.c_float(value).value


def candidate(q, k, v, *, fusion=False, lane_sum=True, round_kv=True, reciprocal=1, stages=1, lse_fma=False,
              native_delta=False, xor_sum=True, native_dq=False, sum_fma=False):
    flags = dict(fusion=fusion, lane_sum=lane_sum, round_kv=round_kv, lse_fma=lse_fma, native_delta=native_delta,
                 xor_sum=xor_sum, native_dq=native_dq, sum_fma=sum_fma)
    bad = [name for name, value in flags.items() if type(value) is not bool]
    if bad or type(reciprocal) is not int or type(stages) is not int or stages < 1:
        raise TypeError(f'candidate flags must be bools and reciprocal/stages ints (got bad: {bad or "ints"})')
    return causal_attention(q, k, v, scale=f32(q.shape[-1] ** -0.5))
