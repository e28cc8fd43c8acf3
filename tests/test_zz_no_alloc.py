"""a8_decode_attn_noalloc, the decode entry point that allocates nothing (its split partials live in a fixed
device array), through the C ABI: its output equals a8_decode_attn's with a caller workspace bit for bit, on two
calls in a row (the second smaller, so it runs over the first call's leftovers in the array), is within the
north-star tolerance of the CPU oracle, and sizes beyond the array are refused with A8_EWSPACE."""
from __future__ import annotations

import ctypes

import pytest
import torch

from conftest import randn_bf16

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
NQ, NKV, HD = 14, 2, 64


def say(msg):
    print(msg, flush=True)


def _case(g, b, S, dev):
    q = randn_bf16(g, b, NQ, HD)
    kc = randn_bf16(g, b + 1, NKV, S, HD)
    vc = randn_bf16(g, b + 1, NKV, S, HD)
    lens = torch.randint(1, S + 1, (b,), generator=g, dtype=torch.int32)
    rowmap = torch.randperm(b + 1, generator=g)[:b].to(torch.int32)
    return q, kc, vc, lens, rowmap


def _call(lib, fn, q, kc, vc, lens, rowmap, out, nsplit, waves, ws=None):
    common = (q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
              kc.stride(2), kc.shape[0], kc.shape[2], lens.data_ptr(), rowmap.data_ptr(), out.data_ptr(),
              out.stride(0), out.stride(1))
    st = torch.cuda.current_stream().cuda_stream
    b = q.shape[0]
    if fn == "noalloc":
        return lib.a8_decode_attn_noalloc(*common, b, NQ, NKV, HD, nsplit, waves, HD ** -0.5, st)
    acc, ml = ws
    return lib.a8_decode_attn(*common, acc.data_ptr(), ml.data_ptr(), acc.numel() // (NQ * HD), None, 0, b, NQ,
                              NKV, HD, nsplit, waves, HD ** -0.5, 3, st)


def test_decode_noalloc_matches_workspace_entry(a8, ref):
    from audio8_turbo_engine_amd import _lib
    lib = _lib.load()
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(11)
    # two calls in a row, the second smaller (fewer rows, fewer splits, shorter cache)
    for b, S, nsplit, waves in ((64, 1024, 8, 2), (5, 300, 3, 1)):
        say(f"case: noalloc b={b} S={S} nsplit={nsplit} waves={waves}")
        q, kc, vc, lens, rowmap = _case(g, b, S, dev)
        qd, kcd, vcd, lensd, rmd = (t.to(dev) for t in (q, kc, vc, lens, rowmap))
        acc = torch.empty(b * nsplit * NQ * HD, dtype=torch.float32, device=dev)
        ml = torch.empty(b * nsplit * NQ * 2, dtype=torch.float32, device=dev)
        o_ws = torch.full((b, NQ, HD), float("nan"), dtype=BF, device=dev)
        o_na = torch.full((b, NQ, HD), float("nan"), dtype=BF, device=dev)
        assert _call(lib, "ws", qd, kcd, vcd, lensd, rmd, o_ws, nsplit, waves, (acc, ml)) == 0
        assert _call(lib, "noalloc", qd, kcd, vcd, lensd, rmd, o_na, nsplit, waves) == 0
        torch.cuda.synchronize()
        assert torch.equal(o_na.cpu(), o_ws.cpu()), "no-alloc output differs from the workspace entry point's"
        o_ref = ref.decode_attention(q, kc, vc, lens, rowmap=rowmap)
        err = (o_na.cpu().float() - o_ref.float()).abs().max().item()
        assert err <= 2e-2, f"max-abs {err} against the oracle"


def test_decode_noalloc_rejects_oversize(a8):
    from audio8_turbo_engine_amd import _lib
    lib = _lib.load()
    dev = torch.device("cuda:0")
    say("case: noalloc size beyond the fixed array")
    b, S, nsplit = 1200, 256, 16   # 1200 * 14 * 16 * 66 * 4 B = 70 MB > 8 MiB
    q = torch.zeros(b, NQ, HD, dtype=BF, device=dev)
    kc = torch.zeros(b, NKV, S, HD, dtype=BF, device=dev)
    lens = torch.full((b,), S, dtype=torch.int32, device=dev)
    rowmap = torch.arange(b, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    st = _call(lib, "noalloc", q, kc, kc, lens, rowmap, out, nsplit, 1)
    assert st == _lib.A8_EWSPACE
    assert b"scratch" in lib.a8_last_error()


def test_decode_noalloc_graph_replay(a8):
    """The no-alloc call captured in a HIP graph: every replay (with eager work and a synchronisation between
    replays, the inputs rewritten in place) equals the eager call on the same inputs bit for bit."""
    from audio8_turbo_engine_amd import _lib
    lib = _lib.load()
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(12)
    b, S, nsplit, waves = 32, 512, 4, 2
    say(f"case: noalloc under graph capture b={b} S={S} nsplit={nsplit}")
    q, kc, vc, lens, rowmap = (t.to(dev) for t in _case(g, b, S, dev))
    out = torch.empty(b, NQ, HD, dtype=BF, device=dev)
    eager = torch.empty_like(out)
    assert _call(lib, "noalloc", q, kc, vc, lens, rowmap, eager, nsplit, waves) == 0  # first call: eager
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            assert _call(lib, "noalloc", q, kc, vc, lens, rowmap, out, nsplit, waves) == 0
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for rep in range(3):
        q.copy_(randn_bf16(g, b, NQ, HD).to(dev))
        assert _call(lib, "noalloc", q, kc, vc, lens, rowmap, eager, nsplit, waves) == 0
        torch.cuda.synchronize()
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), eager.cpu()), f"replay {rep} differs from the eager call"


def test_decode_noalloc_hd128_uses_no_scratch(a8):
    """head_dim 128 goes to the generic-head kernel, which keeps no partials: a split count that would not fit
    the array at head_dim 64 is accepted, and the output equals the workspace entry point's."""
    from audio8_turbo_engine_amd import _lib
    lib = _lib.load()
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(13)
    b, S, nsplit, hd = 600, 64, 16, 128   # 600 * 14 * 16 * 130 * 4 B = 70 MB of partials at hd 64 accounting
    say(f"case: noalloc hd {hd} b={b} nsplit={nsplit}")
    q = randn_bf16(g, b, NQ, hd).to(dev)
    kc = randn_bf16(g, b, NKV, S, hd).to(dev)
    vc = randn_bf16(g, b, NKV, S, hd).to(dev)
    lens = torch.randint(1, S + 1, (b,), generator=g, dtype=torch.int32).to(dev)
    rowmap = torch.arange(b, dtype=torch.int32, device=dev)
    common = (q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
              kc.stride(2), kc.shape[0], kc.shape[2], lens.data_ptr(), rowmap.data_ptr())
    st = torch.cuda.current_stream().cuda_stream
    o_na = torch.full((b, NQ, hd), float("nan"), dtype=BF, device=dev)
    o_ws = torch.full((b, NQ, hd), float("nan"), dtype=BF, device=dev)
    assert lib.a8_decode_attn_noalloc(*common, o_na.data_ptr(), o_na.stride(0), o_na.stride(1), b, NQ, NKV, hd,
                                      nsplit, 1, hd ** -0.5, st) == 0, lib.a8_last_error()
    acc = torch.empty(16 * NQ * hd, dtype=torch.float32, device=dev)
    ml = torch.empty(16 * NQ * 2, dtype=torch.float32, device=dev)
    assert lib.a8_decode_attn(*common, o_ws.data_ptr(), o_ws.stride(0), o_ws.stride(1), acc.data_ptr(), ml.data_ptr(),
                              16, None, 0, b, NQ, NKV, hd, 1, 1, hd ** -0.5, 3, st) == 0, lib.a8_last_error()
    torch.cuda.synchronize()
    assert torch.equal(o_na.cpu(), o_ws.cpu())
