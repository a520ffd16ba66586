"""The no-allocation decode attention entry point (q3_decode_step_attention_noalloc) through the C
ABI: bit-identical outputs and cache writes to q3_decode_step_attention with a caller workspace,
on two calls in a row, the second smaller (the fixed scratch array keeps the first call's
partials, which the second must not read)."""
import pytest
import torch

from _util import seeded

from qwen3_triton import _hip as H

pytestmark = pytest.mark.gpu


def inputs(b, hq, hkv, cap, seed):
    gen = seeded(seed)
    r = lambda *s: torch.randn(*s, generator=gen).to(torch.bfloat16).cuda()  # noqa: E731
    return dict(q=r(b, hq, 128), k=r(b, hkv, 128), v=r(b, hkv, 128), qw=r(128) * 0.1 + 1, kw=r(128) * 0.1 + 1,
                cos=r(b, 128), sin=r(b, 128), ck=r(b, hkv, cap, 128), cv=r(b, hkv, cap, 128))


def run(x, t_len, len_dev, noalloc):
    b, hq, _ = x["q"].shape
    hkv, cap = x["ck"].shape[1], x["ck"].shape[2]
    ck, cv = x["ck"].clone(), x["cv"].clone()
    out = torch.empty_like(x["q"])
    head = [H.BF16, x["q"].data_ptr(), hq * 128, 128, x["k"].data_ptr(), x["v"].data_ptr(), hkv * 128, 128,
            x["qw"].data_ptr(), x["kw"].data_ptr(), 1e-6, x["cos"].data_ptr(), x["sin"].data_ptr(), 128,
            ck.data_ptr(), cv.data_ptr(), hkv * cap * 128, cap * 128, out.data_ptr(), hq * 128, 128]
    tail = [b, hq, hkv, t_len, 0 if len_dev is None else len_dev.data_ptr(), cap, 128, 128 ** -0.5, H.stream()]
    if noalloc:
        H.call("q3_decode_step_attention_noalloc", *head, *tail)
    else:
        span = cap if len_dev is not None else t_len
        ws = torch.empty(H.query("q3_decode_attention_workspace_bytes", b, hq, hkv, span), dtype=torch.uint8,
                         device="cuda")
        H.call("q3_decode_step_attention", *head, ws.data_ptr(), *tail)
    torch.cuda.synchronize()
    return out, ck, cv


@pytest.mark.parametrize("use_len_dev", [False, True])
def test_noalloc_matches_workspace_entry_point(use_len_dev):
    for b, hq, hkv, cap, t_len, seed in [(8, 32, 8, 1280, 1100, 1), (2, 16, 4, 512, 300, 2)]:
        print(f"noalloc decode attention B{b} Hq{hq} Hkv{hkv} cap{cap} T{t_len} len_dev={use_len_dev}", flush=True)
        x = inputs(b, hq, hkv, cap, seed)
        len_dev = torch.tensor([t_len - 1], dtype=torch.int64, device="cuda") if use_len_dev else None
        want = run(x, t_len, len_dev, noalloc=False)
        got = run(x, t_len, len_dev, noalloc=True)
        for a, e, name in zip(got, want, ("out", "cache_k", "cache_v")):
            assert torch.equal(a, e), name
