"""Benchmark: Qwen3-8B decoder layer forward+backward on one MI355X (the headline metric), plus
greedy decode tokens/s.

One "step" = forward + backward of one Qwen3-8B-shape decoder layer (q/k/v/o 4096->4096/1024/1024/
4096, gate/up 4096->12288, down 12288->4096, fused per-head QK-norm + RoPE, GQA causal flash
attention, SwiGLU) over 8192 tokens (batch 4 x seq 2048), bf16 weights/activations, fp32
accumulation, weight gradients included.  Synthetic data: weights N(0, 0.02) (seed 3), hidden
states and upstream gradients N(0, 1).

Printed: one JSON line (rank 0).  ``value`` = tokens/s of the step; ``roofline`` = the dominant
kernel (matrix-core GEMM) timed live with HIP events on its stream inside the timed region;
``cpu_baseline`` = the fp32 CPU oracle's decoder layer on a bounded sample, on this host's cores;
``decode`` = greedy decode tokens/s of the 36-layer Qwen3-8B (random bf16 weights, seed 4): eager
prefill, then one captured decode-step HIP graph replayed per token.
"""
import argparse
import faulthandler
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "qwen3-triton_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 matrix-core peak
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
# HBM bytes per GEMM launch of the layer step, from two rocprofv3 counter passes over
# `bench.py --pmc-probe` (FETCH_SIZE x 2.000 and WRITE_SIZE x 1.000: the factors that make a 1 GiB
# device copy read 1 GiB): every GEMM dispatch of one step (13: the Q/K/V weight gradient runs as two)
# summed and divided by the step's 12 GEMM calls.  Re-measure with those two passes (rocprofv3 --pmc
# FETCH_SIZE / WRITE_SIZE -- python bench.py --pmc-probe) when the GEMM kernels change.
GEMM_TRAFFIC_BYTES_PER_LAUNCH = 1238.6e6 + 204.6e6


def qwen3_8b_config(layers):
    from transformers import Qwen3Config
    return Qwen3Config(vocab_size=151936, hidden_size=4096, intermediate_size=12288, num_hidden_layers=layers,
                       num_attention_heads=32, num_key_value_heads=8, head_dim=128, rope_theta=1e6,
                       rms_norm_eps=1e-6, tie_word_embeddings=False, max_position_embeddings=40960,
                       initializer_range=0.02)


class GemmTimer:
    """Wraps the matrix-core GEMM launcher in every module that calls it: records a HIP event pair on
    the launching stream around every GEMM of the timed region, with its algorithmic FLOPs
    (2*M*N*K)."""

    def __init__(self, modules):
        self.mods = [m for m in modules if hasattr(m, "gemm_nt_into")]
        self.orig = self.mods[0].gemm_nt_into
        assert all(m.gemm_nt_into is self.orig for m in self.mods)
        # the gate/up GEMM with the SwiGLU epilogue (two weights, one launch)
        self.gu_mods = [m for m in modules if hasattr(m, "gate_up_swiglu_into")]
        self.gu_orig = self.gu_mods[0].gate_up_swiglu_into if self.gu_mods else None
        # the same with Y^T stored from the epilogue too (the MLP block's forward)
        self.gt_mods = [m for m in modules if hasattr(m, "gate_up_swiglu_t_into")]
        self.gt_orig = self.gt_mods[0].gate_up_swiglu_t_into if self.gt_mods else None
        # the shared-input projections (q/k/v: up to three weights, one launch)
        self.mu_mods = [m for m in modules if hasattr(m, "gemm_nt_multi_into")]
        self.mu_orig = self.mu_mods[0].gemm_nt_multi_into if self.mu_mods else None
        # the projection GEMM with the residual sum in its epilogue
        self.rs_mods = [m for m in modules if hasattr(m, "gemm_nt_residual_into")]
        self.rs_orig = self.rs_mods[0].gemm_nt_residual_into if self.rs_mods else None
        # the down projection's input-gradient GEMM with the SwiGLU backward epilogue
        self.sb_mods = [m for m in modules if hasattr(m, "swiglu_bwd_gemm_into")]
        self.sb_orig = self.sb_mods[0].swiglu_bwd_gemm_into if self.sb_mods else None
        self.records = []
        self.active = False

    def __enter__(self):
        import torch
        orig = self.orig

        def timed(a, lda, bnk, ldb, out, m, n, k, **kw):
            if not self.active:
                return orig(a, lda, bnk, ldb, out, m, n, k, **kw)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            orig(a, lda, bnk, ldb, out, m, n, k, **kw)
            e.record()
            self.records.append((s, e, 2.0 * m * n * k))

        def timed_gu(x, wg, wu, g, u, y, m, n, k):
            if not self.active:
                return self.gu_orig(x, wg, wu, g, u, y, m, n, k)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            self.gu_orig(x, wg, wu, g, u, y, m, n, k)
            e.record()
            self.records.append((s, e, 2.0 * 2 * m * n * k))

        def timed_gt(x, wg, wu, g, u, y, yt, m, n, k):
            if not self.active:
                return self.gt_orig(x, wg, wu, g, u, y, yt, m, n, k)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            self.gt_orig(x, wg, wu, g, u, y, yt, m, n, k)
            e.record()
            self.records.append((s, e, 2.0 * 2 * m * n * k))

        def timed_mu(a, weights, outs, m, k):
            if not self.active:
                return self.mu_orig(a, weights, outs, m, k)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            self.mu_orig(a, weights, outs, m, k)
            e.record()
            self.records.append((s, e, 2.0 * m * k * sum(w.shape[0] for w in weights)))

        def timed_sb(dy, wt, g, u, dg, du, dgt, dut, m, n, k):
            if not self.active:
                return self.sb_orig(dy, wt, g, u, dg, du, dgt, dut, m, n, k)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            self.sb_orig(dy, wt, g, u, dg, du, dgt, dut, m, n, k)
            e.record()
            self.records.append((s, e, 2.0 * m * n * k))

        def timed_rs(a, lda, bnk, ldb, res, out, m, n, k):
            if not self.active:
                return self.rs_orig(a, lda, bnk, ldb, res, out, m, n, k)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            self.rs_orig(a, lda, bnk, ldb, res, out, m, n, k)
            e.record()
            self.records.append((s, e, 2.0 * m * n * k))

        for m in self.mods:
            m.gemm_nt_into = timed
        for m in self.rs_mods:
            m.gemm_nt_residual_into = timed_rs
        for m in self.sb_mods:
            m.swiglu_bwd_gemm_into = timed_sb
        for m in self.gu_mods:
            m.gate_up_swiglu_into = timed_gu
        for m in self.gt_mods:
            m.gate_up_swiglu_t_into = timed_gt
        for m in self.mu_mods:
            m.gemm_nt_multi_into = timed_mu
        return self

    def __exit__(self, *exc):
        for m in self.mods:
            m.gemm_nt_into = self.orig
        for m in self.gu_mods:
            m.gate_up_swiglu_into = self.gu_orig
        for m in self.gt_mods:
            m.gate_up_swiglu_t_into = self.gt_orig
        for m in self.mu_mods:
            m.gemm_nt_multi_into = self.mu_orig
        for m in self.sb_mods:
            m.swiglu_bwd_gemm_into = self.sb_orig
        for m in self.rs_mods:
            m.gemm_nt_residual_into = self.rs_orig

    def summary(self):
        ms = sum(s.elapsed_time(e) for s, e, _ in self.records)
        flops = sum(f for _, _, f in self.records)
        n = len(self.records)
        return n, ms, flops


def decoder_layer_bench(steps, warmup):
    import torch
    from qwen3_triton.components import DecoderLayer
    from qwen3_triton.configuration import OptimizationOptions
    from qwen3_triton.kernels import linear as linear_mod, mlp_precision, lm_head_ce
    from qwen3_triton.kernels.rotary import rotary_tables
    from qwen3_triton._model import rope_theta

    torch.manual_seed(3)
    cfg = qwen3_8b_config(1)
    layer = DecoderLayer(cfg, OptimizationOptions()).to(device="cuda", dtype=torch.bfloat16)
    gen = torch.Generator(device="cuda").manual_seed(3)
    with torch.no_grad():
        for name, p in layer.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.normal_(0.0, 0.02, generator=gen)
    b, s, h = 4, 2048, 4096
    x = torch.randn(b, s, h, device="cuda", dtype=torch.bfloat16, generator=gen).requires_grad_()
    dy = torch.randn(b, s, h, device="cuda", dtype=torch.bfloat16, generator=gen)
    pos = torch.arange(s, device="cuda", dtype=torch.int64).repeat(b, 1)
    inv = (1.0 / (rope_theta(cfg) ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))).cuda()
    cos, sin = rotary_tables(pos, inv, torch.bfloat16)
    params = list(layer.parameters())

    def step():
        x.grad = None
        for p in params:
            p.grad = None
        y = layer(x, (cos, sin))
        y.backward(dy)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    with GemmTimer([linear_mod, mlp_precision, lm_head_ce]) as gt:
        gt.active = True
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record()
        for _ in range(steps):
            step()
        end.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        gt.active = False
    ms_step = start.elapsed_time(end) / steps
    n, gemm_ms, gemm_flops = gt.summary()
    tokens = b * s
    # algorithmic matrix-core work of the step: projections 3x (fwd, dX, dW) + causal attention
    gemm_step_flops = 3 * 2 * tokens * (h * (4096 + 1024 + 1024 + 4096) + 3 * h * 12288)
    attn_step_flops = 3.5 * 2 * b * 32 * s * s * 128   # causal fwd (1x) + bwd (2.5x)
    return {
        "tokens": tokens, "ms_per_step": ms_step, "wall_s": wall,
        "tokens_per_s": tokens / (ms_step * 1e-3),
        "gemm_launches": n, "gemm_ms_per_step": gemm_ms / steps, "gemm_flops_per_step": gemm_flops / steps,
        "gemm_tflops": gemm_flops / (gemm_ms * 1e-3) / 1e12 if gemm_ms > 0 else 0.0,
        "algorithmic_tflops_per_step": (gemm_step_flops + attn_step_flops) / 1e12,
        "step_tflops": (gemm_step_flops + attn_step_flops) / (ms_step * 1e-3) / 1e12,
    }


def cpu_baseline(seconds_budget=20.0):
    """fp32 CPU oracle decoder layer forward+backward on batch 1 x 512 tokens (same shapes and
    weight distribution), median of timed repetitions after one warm-up."""
    import torch
    import oracle as O
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    oc = O.OracleConfig(vocab_size=16, hidden_size=4096, intermediate_size=12288, num_hidden_layers=1,
                        num_attention_heads=32, num_key_value_heads=8, head_dim=128)
    params = {k: v.requires_grad_() for k, v in O.init_params(oc, seed=3).items() if k.startswith("model.layers.0.")}
    tokens = 512
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(1, tokens, 4096, generator=gen).requires_grad_()
    dy = torch.randn(1, tokens, 4096, generator=gen)
    cos, sin = O.rotary_tables_reference(torch.arange(tokens)[None], O.rope_inv_freq(1e6, 128))

    def run():
        for p in params.values():
            p.grad = None
        y = O.decoder_layer_reference(x, params, "model.layers.0.", oc, cos, sin)
        y.backward(dy)

    t0 = time.perf_counter()
    run()
    first = time.perf_counter() - t0
    reps = max(1, min(5, int(seconds_budget / max(first, 1e-3))))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {"value": tokens / med, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"fp32 oracle decoder layer fwd+bwd, batch 1 x {tokens} tokens, median of {reps}"}


def decode_bench(batch, prompt, new_tokens):
    """Greedy decode of the 36-layer Qwen3-8B: eager prefill (timed on a second, warm pass), then one
    captured decode-step graph replayed ``new_tokens`` times (the cache length lives on the device).
    The decode rate is timed with HIP events around the replays only."""
    import torch
    from qwen3_triton.inference import DecodeSession, TritonQwen3Inference
    cfg = qwen3_8b_config(36)
    model = TritonQwen3Inference.random_init(cfg, seed=4, std=0.02, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(4)
    ids = torch.randint(0, cfg.vocab_size, (batch, prompt), device="cuda", generator=gen)
    sess = DecodeSession(model, batch, prompt + new_tokens + 1)
    sess.prefill(ids)    # cold pass (allocations, first launches), then the timed prefill
    sess.reset()
    torch.cuda.synchronize()
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record()
    sess.prefill(ids)
    s1.record()
    sess.step()          # one eager step (warms the step's allocations)
    sess.capture()
    torch.cuda.synchronize()
    prefill_ms = s0.elapsed_time(s1)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    steps = new_tokens - 1
    e0.record()
    for _ in range(steps):
        sess.step()
    e1.record()
    torch.cuda.synchronize()
    per_step_ms = e0.elapsed_time(e1) / steps
    layer_bytes = 36 * 2 * (4096 * (4096 + 1024 + 1024 + 4096) + 3 * 4096 * 12288)
    head_bytes = 2 * 4096 * 151936
    mean_ctx = prompt + 1 + new_tokens / 2
    kv_bytes = 36 * 2 * 8 * 128 * 2 * mean_ctx * batch
    step_bytes = layer_bytes + head_bytes + kv_bytes
    del sess, model
    torch.cuda.empty_cache()
    return {"batch": batch, "prompt": prompt, "new_tokens": new_tokens, "prefill_ms": round(prefill_ms, 3),
            "ms_per_step": round(per_step_ms, 4), "tokens_per_s": round(batch / (per_step_ms * 1e-3), 1),
            "hbm_gb_per_step": round(step_bytes / 1e9, 3),
            "hbm_gbs": round(step_bytes / (per_step_ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(step_bytes / (per_step_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}


def lm_head_ce_bench(steps=3, warmup=1):
    """Fused LM-head + causal CE of config #4: hidden [4, 2048, 4096] N(0,1), W [151936, 4096]
    N(0, 0.02), labels uniform over the vocabulary with 5 % set to -100 (seed 3); forward + backward.
    Algorithmic work: logits, dX and dW, 3 x 2*T*H*V FLOPs (the forward keeps the bf16 logits, so the
    backward runs no second logits GEMM)."""
    import torch
    from qwen3_triton.kernels.lm_head_ce import lm_head_cross_entropy
    b, s, h, v = 4, 2048, 4096, 151936
    gen = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(b, s, h, device="cuda", dtype=torch.bfloat16, generator=gen).requires_grad_()
    w = (torch.randn(v, h, device="cuda", dtype=torch.bfloat16, generator=gen) * 0.02).requires_grad_()
    labels = torch.randint(0, v, (b, s), device="cuda", generator=gen)
    drop = torch.rand(b, s, device="cuda", generator=gen) < 0.05
    labels = torch.where(drop, torch.full_like(labels, -100), labels)

    def step():
        x.grad = None
        w.grad = None
        lm_head_cross_entropy(x, w, labels).backward()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = 3 * 2.0 * b * s * h * v
    del x, w
    torch.cuda.empty_cache()
    return {"tokens": b * s, "vocab": v, "ms_per_step": round(ms, 3), "tokens_per_s": round(b * s / (ms * 1e-3), 1),
            "algorithmic_tflop_per_step": round(flops / 1e12, 2),
            "achieved_tflops": round(flops / (ms * 1e-3) / 1e12, 1),
            "frac": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}


def _event_ms(fn, reps):
    import torch
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def attention_bench(reps=10):
    """Config #3: GQA causal flash attention (32 query / 8 KV heads, head_dim 128, bf16, seed 2) at
    B4 x S2048 and B1 x S8192.  Forward = the V^T copy + the flash kernel; backward = delta, the K^T
    copy, dQ and dK/dV (the whole op as the autograd backward runs it).  Algorithmic work: causal
    forward 2 * 2 * B * Hq * S^2 / 2 * D FLOP, backward 2.5 x that."""
    import torch
    from qwen3_triton.kernels import _ops
    out = {}
    gen = torch.Generator(device="cuda").manual_seed(2)
    for b, s in ((4, 2048), (1, 8192)):
        q = torch.randn(b, s, 32, 128, device="cuda", dtype=torch.bfloat16, generator=gen).transpose(1, 2)
        k = torch.randn(b, s, 8, 128, device="cuda", dtype=torch.bfloat16, generator=gen).transpose(1, 2)
        v = torch.randn(b, s, 8, 128, device="cuda", dtype=torch.bfloat16, generator=gen).transpose(1, 2)
        do = torch.randn(b, s, 32, 128, device="cuda", dtype=torch.bfloat16, generator=gen).transpose(1, 2)
        sc = 128 ** -0.5
        o, lse = _ops.attention_fwd(q, k, v, sc)
        f_ms = _event_ms(lambda: _ops.attention_fwd(q, k, v, sc), reps)
        b_ms = _event_ms(lambda: _ops.attention_bwd(q, k, v, o, lse, do, sc), reps)
        fwd_flops = 2 * 2 * b * 32 * s * s / 2 * 128
        f_tf, b_tf = fwd_flops / (f_ms * 1e-3) / 1e12, 2.5 * fwd_flops / (b_ms * 1e-3) / 1e12
        out[f"b{b}_s{s}"] = {"fwd_ms": round(f_ms, 4), "fwd_tflops": round(f_tf, 1),
                             "fwd_frac": round(f_tf / PEAK_BF16_TFLOPS, 4), "bwd_ms": round(b_ms, 4),
                             "bwd_tflops": round(b_tf, 1), "bwd_frac": round(b_tf / PEAK_BF16_TFLOPS, 4)}
        del q, k, v, do, o, lse
    torch.cuda.empty_cache()
    return out


def bandwidth_bench(reps=20):
    """Config #2: the bandwidth-bound ops at Qwen3-8B shape, bf16 (seed 1): RMSNorm on [8192, 4096],
    fused per-head QK-norm + RoPE on Q [8192, 32, 128] and K [8192, 8, 128] (each alone, and both in
    one launch as the layer runs them), RoPE on Q, SwiGLU on
    [8192, 12288].  Kernel launches on preallocated buffers; achieved = algorithmic HBM bytes (each
    operand read or written once: x/y 2 B per element, plus weights and rotary tables) / time."""
    import torch
    from qwen3_triton import _hip as H
    from qwen3_triton.kernels import _ops
    gen = torch.Generator(device="cuda").manual_seed(1)
    bf = torch.bfloat16
    st = H.stream()
    res = {}

    def rec(name, ms, nbytes):
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"us": round(ms * 1e3, 2), "gb": round(nbytes / 1e9, 4), "gbs": round(gbs, 1),
                     "frac": round(gbs / PEAK_HBM_GBS, 4)}

    t, h = 8192, 4096
    x = torch.randn(t, h, device="cuda", dtype=bf, generator=gen)
    w = (1 + 0.1 * torch.randn(h, device="cuda", generator=gen)).to(bf)
    y, dy, dx = torch.empty_like(x), torch.randn(t, h, device="cuda", dtype=bf, generator=gen), torch.empty_like(x)
    dw = torch.empty_like(w)
    ws = H.workspace(H.query("q3_rmsnorm_bwd_workspace_bytes", t, h), x.device)
    rec("rmsnorm_fwd", _event_ms(lambda: H.call("q3_rmsnorm_fwd", H.BF16, x.data_ptr(), w.data_ptr(), y.data_ptr(), t,
                                                h, 1e-6, st), reps), 2 * 2 * t * h)
    rec("rmsnorm_bwd", _event_ms(lambda: H.call("q3_rmsnorm_bwd", H.BF16, x.data_ptr(), w.data_ptr(), dy.data_ptr(),
                                                dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), t, h, 1e-6, st), reps),
        3 * 2 * t * h)
    del x, y, dy, dx
    pos = torch.arange(2048, device="cuda").repeat(4, 1)
    inv = (1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))).cuda()
    cos, sin = _ops.rope_tables(pos, inv, bf)
    tab = 2 * 2 * t * 128
    keep = {}
    for name, heads in (("q", 32), ("k", 8)):
        xq = torch.randn(4, 2048, heads, 128, device="cuda", dtype=bf, generator=gen)
        wq = (1 + 0.1 * torch.randn(128, device="cuda", generator=gen)).to(bf)
        yq, dyq, dxq, dwq = torch.empty_like(xq), torch.randn_like(xq), torch.empty_like(xq), torch.empty_like(wq)
        wsq = H.workspace(H.query("q3_norm_rope_bwd_workspace_bytes", t, heads, 128), xq.device)
        n = xq.numel()
        rec(f"qk_norm_rope_fwd_{name}", _event_ms(lambda: H.call(
            "q3_norm_rope_fwd", H.BF16, xq.data_ptr(), wq.data_ptr(), cos.data_ptr(), sin.data_ptr(), yq.data_ptr(), t,
            heads, 128, 1e-6, st), reps), 2 * 2 * n + tab)
        rec(f"qk_norm_rope_bwd_{name}", _event_ms(lambda: H.call(
            "q3_norm_rope_bwd", H.BF16, xq.data_ptr(), wq.data_ptr(), cos.data_ptr(), sin.data_ptr(), dyq.data_ptr(),
            dxq.data_ptr(), dwq.data_ptr(), wsq.data_ptr(), t, heads, 128, 1e-6, st), reps), 3 * 2 * n + tab)
        if name == "q":
            rec("rope_fwd_q", _event_ms(lambda: H.call("q3_rope_apply", H.BF16, xq.data_ptr(), cos.data_ptr(),
                                                       sin.data_ptr(), yq.data_ptr(), 4, 2048, heads, 128, 0, 0, st),
                                        reps), 2 * 2 * n + tab)
        keep[name] = (xq, wq, yq, dyq, dxq)
    # the layer's Q and K heads in one launch per direction (q3_norm_rope_qk_*)
    (xq, wq, yq, dyq, dxq), (xk, wk, yk, dyk, dxk) = keep["q"], keep["k"]
    dwqk = torch.empty(2, 128, device="cuda", dtype=bf)
    wsqk = H.workspace(H.query("q3_norm_rope_qk_bwd_workspace_bytes", t, 32, 8, 128), xq.device)
    n = xq.numel() + xk.numel()
    rec("qk_norm_rope_fwd_qk", _event_ms(lambda: H.call(
        "q3_norm_rope_qk_fwd", H.BF16, xq.data_ptr(), xk.data_ptr(), wq.data_ptr(), wk.data_ptr(), cos.data_ptr(),
        sin.data_ptr(), yq.data_ptr(), yk.data_ptr(), t, 32, 8, 128, 1e-6, st), reps), 2 * 2 * n + tab)
    rec("qk_norm_rope_bwd_qk", _event_ms(lambda: H.call(
        "q3_norm_rope_qk_bwd", H.BF16, xq.data_ptr(), xk.data_ptr(), wq.data_ptr(), wk.data_ptr(), cos.data_ptr(),
        sin.data_ptr(), dyq.data_ptr(), dyk.data_ptr(), dxq.data_ptr(), dxk.data_ptr(), dwqk.data_ptr(),
        wsqk.data_ptr(), t, 32, 8, 128, 1e-6, st), reps), 3 * 2 * n + tab)
    del keep, xq, yq, dyq, dxq, xk, yk, dyk, dxk
    g = torch.randn(t, 12288, device="cuda", dtype=bf, generator=gen)
    u = torch.randn(t, 12288, device="cuda", dtype=bf, generator=gen)
    dyg, yg, dg, du = torch.randn_like(g), torch.empty_like(g), torch.empty_like(g), torch.empty_like(g)
    n = g.numel()
    rec("swiglu_fwd", _event_ms(lambda: H.call("q3_swiglu_fwd", H.BF16, g.data_ptr(), u.data_ptr(), yg.data_ptr(), n,
                                               st), reps), 3 * 2 * n)
    rec("swiglu_bwd", _event_ms(lambda: H.call("q3_swiglu_bwd", H.BF16, g.data_ptr(), u.data_ptr(), dyg.data_ptr(),
                                               dg.data_ptr(), du.data_ptr(), n, st), reps), 5 * 2 * n)
    del g, u, dyg, yg, dg, du
    torch.cuda.empty_cache()
    return res


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main():
    faulthandler.enable()
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-layer", action="store_true", help="skip the decoder-layer step (profiling decode)")
    ap.add_argument("--no-lm-head", action="store_true", help="skip the fused LM-head + CE step")
    ap.add_argument("--no-ops", action="store_true", help="skip the per-op attention / bandwidth measurements")
    ap.add_argument("--decode-tokens", type=int, default=256)
    ap.add_argument("--decode-batches", default="1,8", help="comma list of decode batches among 1 and 8")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="run one warm-up + one decoder-layer step and a 1 GiB device copy, then exit (the "
                         "workload of the FETCH_SIZE / WRITE_SIZE counter passes behind roofline.traffic)")
    args = ap.parse_args()
    if args.pmc_probe:
        import torch
        decoder_layer_bench(1, 1)
        src = torch.empty(1 << 29, device="cuda", dtype=torch.bfloat16).fill_(1.0)   # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(2):
            dst.copy_(src)   # calibration: reads and writes exactly 1 GiB
        torch.cuda.synchronize()
        log("pmc probe done")
        return
    if args.gpus != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (collectives are out of scope); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    from qwen3_triton import _hip
    _hip.load()

    if args.no_layer:
        layer = {"tokens_per_s": float("nan"), "ms_per_step": float("nan"), "tokens": 8192, "gemm_tflops": 0.0,
                 "gemm_launches": 0, "gemm_flops_per_step": 0.0, "algorithmic_tflops_per_step": 0.0,
                 "step_tflops": 0.0}
    else:
        log("decoder layer fwd+bwd")
        layer = decoder_layer_bench(args.steps, args.warmup)
        log(f"decoder layer: {layer['ms_per_step']:.3f} ms/step")
    result = {
        "metric": "decoder-layer fwd+bwd tokens/s @Qwen3-8B shape, 1 GPU, % roofline; decode tok/s",
        "value": round(layer["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(layer["ms_per_step"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random N(0,0.02) weights, N(0,1) hidden states and upstream gradients)",
        "config": {"workload": "qwen3-8b decoder layer fwd+bwd (config #4 layer)", "model": "Qwen3-8B layer",
                   "global_batch": 4, "seq_len": 2048, "tokens_per_step": layer["tokens"], "parallelism": "none"},
        "roofline": {"bound": "mfma", "kernel": "gemm_nt_v4_kernel (bf16 MFMA GEMM)",
                     "achieved": round(layer["gemm_tflops"], 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(layer["gemm_tflops"] / PEAK_BF16_TFLOPS, 4), "traffic": GEMM_TRAFFIC_BYTES_PER_LAUNCH,
                     "launches_per_step": layer["gemm_launches"] // args.steps,
                     "flops_per_launch": layer["gemm_flops_per_step"] / max(1, layer["gemm_launches"] // args.steps)},
        "step_roofline": {"algorithmic_tflop_per_step": round(layer["algorithmic_tflops_per_step"], 3),
                          "achieved_tflops": round(layer["step_tflops"], 1),
                          "frac": round(layer["step_tflops"] / PEAK_BF16_TFLOPS, 4)},
    }
    if not args.no_ops:
        log("attention (config #3) and bandwidth-bound ops (config #2)")
        result["attention"] = attention_bench()
        result["bandwidth_ops"] = bandwidth_bench()
    if not args.no_lm_head:
        log("fused LM-head CE fwd+bwd")
        result["lm_head_ce"] = lm_head_ce_bench()
    if not args.no_decode:
        log("decode")
        try:
            prompts = {1: 2048, 8: 1024}
            result["decode"] = {f"b{b}": decode_bench(b, prompts[b], args.decode_tokens)
                                for b in (int(x) for x in args.decode_batches.split(","))}
        except Exception as exc:  # report, do not hide the layer result
            result["decode"] = {"error": repr(exc)}
    if not args.no_cpu_baseline:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
