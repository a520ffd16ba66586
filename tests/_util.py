"""Shared helpers for the parity tests (tolerances follow the north-star gates)."""
import torch


def seeded(seed):
    return torch.Generator().manual_seed(seed)


def randn(*shape, gen, dtype=torch.float32, scale=1.0, shift=0.0):
    return (torch.randn(*shape, generator=gen) * scale + shift).to(dtype)


def to_dev(*ts):
    return [t.cuda() for t in ts]


def max_rel(actual, expected):
    """max |a-e| / max |e| (the 'max relative error' of the bf16 forward gate, 2e-2)."""
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    return float((a - e).abs().max() / e.abs().max().clamp_min(1e-30))


def cosine(actual, expected):
    a = actual.detach().double().cpu().flatten()
    e = expected.detach().double().cpu().flatten()
    return float(torch.dot(a, e) / (a.norm() * e.norm()).clamp_min(1e-300))


def tol_for(dtype):
    return {torch.float32: 1e-5, torch.float16: 3e-3, torch.bfloat16: 2e-2}[dtype]
