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


def test_noalloc_first_call_under_graph_capture():
    """Collected first in this file, so in a fresh process the entry point's first call on the device
    (the one that looks up the scratch array's address) happens inside ``torch.cuda.graph`` capture.
    The graph is replayed with new query / key / value contents and new device-resident lengths, each
    replay against the workspace entry point called eagerly on the same inputs, bit for bit."""
    b, hq, hkv, cap = 4, 32, 8, 1280
    x = inputs(b, hq, hkv, cap, 7)
    ck, cv = x["ck"].clone(), x["cv"].clone()
    out = torch.empty_like(x["q"])
    len_dev = torch.tensor([1099], dtype=torch.int64, device="cuda")
    args = [H.BF16, x["q"].data_ptr(), hq * 128, 128, x["k"].data_ptr(), x["v"].data_ptr(), hkv * 128, 128,
            x["qw"].data_ptr(), x["kw"].data_ptr(), 1e-6, x["cos"].data_ptr(), x["sin"].data_ptr(), 128,
            ck.data_ptr(), cv.data_ptr(), hkv * cap * 128, cap * 128, out.data_ptr(), hq * 128, 128,
            b, hq, hkv, 1100, len_dev.data_ptr(), cap, 128, 128 ** -0.5]
    torch.cuda.synchronize()
    print("noalloc decode attention captured in a graph (first call on the device)", flush=True)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        H.call("q3_decode_step_attention_noalloc", *args, stream.cuda_stream)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for i, length in enumerate([1099, 700, 1200, 5]):
        print(f"noalloc graph replay {i}: length {length}", flush=True)
        fresh = inputs(b, hq, hkv, cap, 20 + i)
        for name in ("q", "k", "v"):
            x[name].copy_(fresh[name])
        ck.copy_(x["ck"])
        cv.copy_(x["cv"])
        len_dev.fill_(length)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = run(x, length + 1, torch.tensor([length], dtype=torch.int64, device="cuda"), noalloc=False)
        for a, e, name in zip((out, ck, cv), want, ("out", "cache_k", "cache_v")):
            assert torch.equal(a, e), f"replay {i} {name}"


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
