"""``qwen3_triton/kernels/attention_precision.py:147-182`` (``candidate``).

The reference's flags select SM86 rounding/reduction orders (exp2 vs exp, reverse tile order,
4-lane sums, reciprocal PTX, split dQ).  On gfx950 the flash kernels have one schedule: base-2
online softmax, fp32 accumulation, deterministic GQA reduction.  The flags are accepted so the
call signature is unchanged; they select nothing.
"""
from .attention import causal_attention


def candidate(q, k, v, *, fusion=False, lane_sum=True, round_kv=True, reciprocal=1, stages=1, lse_fma=True,
              native_delta=True, xor_sum=True, native_dq=True, sum_fma=True):
    return causal_attention(q, k, v, scale=q.shape[-1] ** -0.5)
