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
    if float(e.abs().max()) == 0.0:
        return float(a.abs().max())
    return float((a - e).abs().max() / e.abs().max())


def cosine(actual, expected):
    """Cosine similarity; an all-zero expected tensor counts as 1.0 when the actual one is ~0 too."""
    a = actual.detach().double().cpu().flatten()
    e = expected.detach().double().cpu().flatten()
    if float(e.norm()) == 0.0:
        return 1.0 if float(a.abs().max()) < 1e-3 else 0.0
    return float(torch.dot(a, e) / (a.norm() * e.norm()).clamp_min(1e-300))


def tol_for(dtype):
    return {torch.float32: 1e-5, torch.float16: 3e-3, torch.bfloat16: 2e-2}[dtype]
