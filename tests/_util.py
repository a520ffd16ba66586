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


def greedy_parity(model, p32, cfg, prompt, steps, *, label=""):
    """Greedy decoding on the GPU against the fp32 KV-cached oracle on the same (bf16-rounded)
    weights; returns the oracle's free-running tokens [B, steps].

    1. Teacher forcing: the GPU model is fed the ORACLE's tokens through its KV cache, so both runs
       see the same context at every step.  Each step's last-position logits must meet the bf16
       forward gate (normwise max-rel <= 2e-2).  The GPU argmax must equal the oracle's token, or
       else the mismatch must be explained by the measured error: the oracle logit of the GPU's
       pick lies within 2 * err of the oracle's top logit, err = max |GPU - oracle| over that
       row's logits.  So every step whose oracle top-2 margin exceeds 2 * err (a decisive step)
       must match exactly.  At least 75 % of all (row, step) pairs must match exactly, so the check
       cannot pass vacuously; the counts are printed.
    2. Free running: ``generate`` must reproduce the oracle's tokens in every row up to the row's
       first teacher-forced mismatch (all of them when there is none): until then both runs see
       the same context, and the kernels are deterministic.
    """
    import oracle as O
    b, s = prompt.shape
    exp_tok, exp_logits = O.cached_decode_reference(prompt, p32, cfg, steps)
    cache = model.new_cache(b, s + steps)
    dev = prompt.cuda()
    got = [model(dev, past_key_values=cache).logits[:, -1].float().cpu()]
    for t in range(steps - 1):
        got.append(model(exp_tok[:, t:t + 1].cuda(), past_key_values=cache).logits[:, -1].float().cpu())
    got = torch.stack(got, dim=1)
    exact = torch.zeros(b, steps, dtype=torch.bool)
    n_decisive, errs = 0, []
    for r in range(b):
        for t in range(steps):
            e, a = exp_logits[r, t], got[r, t]
            assert max_rel(a, e) <= 2e-2, f"{label} row {r} step {t}: logits max-rel {max_rel(a, e):.3e}"
            err = float((a.double() - e.double()).abs().max())
            errs.append(err)
            top2 = e.topk(2).values
            n_decisive += float(top2[0] - top2[1]) > 2 * err
            pick, want = int(a.argmax()), int(exp_tok[r, t])
            exact[r, t] = pick == want
            gap = float(e[want] - e[pick])
            assert pick == want or gap <= 2 * err, \
                f"{label} row {r} step {t}: GPU picks {pick}, {gap:.4f} below the oracle's {want} (err {err:.4f})"
    n_exact = int(exact.sum())
    errs = torch.tensor(errs)
    print(f"{label}: {n_exact}/{b * steps} (row, step) tokens exact, {n_decisive} decisive "
          f"(margin > 2 x max logit error; median error {float(errs.median()):.4f})", flush=True)
    assert n_exact >= 0.75 * b * steps, f"{label}: only {n_exact}/{b * steps} tokens exact"
    free = model.generate(dev, max_new_tokens=steps, eos_token_id=[], pad_token_id=0).cpu()
    for r in range(b):
        for t in range(steps):
            if not exact[r, t]:
                break
            assert int(free[r, s + t]) == int(exp_tok[r, t]), f"{label} free-running row {r} step {t}"
    return exp_tok
