"""GPU parity of the single-launch balanced decode (DecodeAttention mode "flat" -> a8_decode_attn_flat /
a8_store_decode_flat) against the CPU oracle: forced grids from one workgroup up (so rows spread over many
wavefronts and are merged in the launch), ragged / empty / unmapped rows, repeatability, the counters left
at zero, the fused store bit for bit against the two calls, and graph replays.
Bar: max-abs <= 2e-2 on the bf16 outputs."""
from __future__ import annotations

import pytest
import torch

from conftest import randn_bf16

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
NQ, NKV, HD = 14, 2, 64
W = (NQ + 2 * NKV) * HD
TOL = 2e-2


def say(msg):
    print(msg, flush=True)


def maxabs(a, b):
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


def bits(t):
    return t.view(torch.int16)


def _ragged(seed, b, rows, S):
    g = torch.Generator().manual_seed(seed)
    q = randn_bf16(g, b, NQ, HD)
    kc, vc = randn_bf16(g, rows, NKV, S, HD), randn_bf16(g, rows, NKV, S, HD)
    lens = torch.randint(1, S + 1, (b,), generator=g).int()
    return g, q, kc, vc, lens


@pytest.mark.parametrize("grid", [1, 2, 3, 5, 16, 64, 256])
def test_flat_grids_ragged(a8, ref, dev, grid):
    """Ragged rows incl. 0 / 1 / 64 / 65 keys, one past the cache (clamped), unmapped cache rows (NaN, like an
    empty row); every grid gives the oracle's answer, the same bits twice, and leaves the counters at zero."""
    say(f"case: flat decode grid={grid}")
    b, rows, S = 21, 9, 1500
    g, q, kc, vc, lens = _ragged(31, b, rows, S)
    lens[:7] = torch.tensor([0, 1, 64, 65, 1500, 0, 2000], dtype=torch.int32)
    rowmap = torch.randint(0, rows, (b,), generator=g).int()
    rowmap[7], rowmap[8] = -1, rows                                   # outside the cache
    want = ref.decode_attention(q, kc, vc, lens.clamp(max=S), rowmap=rowmap.clamp(0, rows - 1))
    att = a8.DecodeAttention(4096, NQ, NKV, HD, 16, dev)             # 2 partial slots per wave up to grid 1024
    att.force_flat = grid
    assert att.schedule(b, S) == ("flat", (grid,))
    outs = []
    for _ in range(2):
        out = torch.empty(b, NQ, HD, dtype=BF, device=dev)
        att(q.to(dev), kc.to(dev), vc.to(dev), lens.to(dev), out, rowmap=rowmap.to(dev))
        torch.cuda.synchronize()
        outs.append(out.cpu())
        assert int(att.counters.abs().sum()) == 0
    assert torch.equal(bits(outs[0]), bits(outs[1]))
    o = outs[0]
    for r in (0, 5, 7, 8):
        assert torch.isnan(o[r].float()).all(), r
    ok = [r for r in range(b) if r not in (0, 5, 7, 8)]
    assert maxabs(o[ok], want[ok]) <= TOL


@pytest.mark.parametrize("grid", [1, 4, 16, 37])
def test_flat_long_row_many_waves(a8, ref, dev, grid):
    """One 2048-key row next to short ones: with 4 grid waves over ~70 tiles the long row's two units are
    spread over up to 64 wavefronts whose ranges start and end inside units (first / last segment slots)."""
    say(f"case: flat decode long row, grid={grid}")
    g = torch.Generator().manual_seed(32)
    b, S = 4, 2048
    q = randn_bf16(g, b, NQ, HD)
    kc, vc = randn_bf16(g, b, NKV, S, HD), randn_bf16(g, b, NKV, S, HD)
    lens = torch.tensor([70, 2048, 3, 130], dtype=torch.int32)
    want = ref.decode_attention(q, kc, vc, lens)
    att = a8.DecodeAttention(4096, NQ, NKV, HD, 16, dev)
    att.force_flat = grid
    out = torch.empty(b, NQ, HD, dtype=BF, device=dev)
    att(q.to(dev), kc.to(dev), vc.to(dev), lens.to(dev), out)
    torch.cuda.synchronize()
    assert int(att.counters.abs().sum()) == 0
    assert maxabs(out, want) <= TOL


def test_flat_edge_values(a8, dev):
    """L = 1 gives V[0] exactly; lens past the cache equal lens = S."""
    say("case: flat decode L=1 / lens > S")
    g = torch.Generator().manual_seed(33)
    b, S = 4, 96
    q = randn_bf16(g, b, NQ, HD)
    kc, vc = randn_bf16(g, b, NKV, S, HD), randn_bf16(g, b, NKV, S, HD)
    att = a8.DecodeAttention(256, NQ, NKV, HD, 16, dev)
    for grid in (1, 3):
        att.force_flat = grid
        out = torch.empty(b, NQ, HD, dtype=BF, device=dev)
        att(q.to(dev), kc.to(dev), vc.to(dev), torch.ones(b, dtype=torch.int32, device=dev), out)
        torch.cuda.synchronize()
        for i in range(b):
            assert torch.equal(out[i, :7].cpu(), vc[i, 0, 0].expand(7, HD))
            assert torch.equal(out[i, 7:].cpu(), vc[i, 1, 0].expand(7, HD))
        full = torch.empty_like(out)
        over = torch.empty_like(out)
        att(q.to(dev), kc.to(dev), vc.to(dev), torch.full((b,), S, dtype=torch.int32, device=dev), full)
        att(q.to(dev), kc.to(dev), vc.to(dev), torch.full((b,), S + 500, dtype=torch.int32, device=dev), over)
        torch.cuda.synchronize()
        assert torch.equal(bits(full.cpu()), bits(over.cpu()))


@pytest.mark.parametrize("b,S", [(1, 512), (64, 4096), (384, 10), (192, 10), (7, 100), (300, 3000)])
def test_flat_default_shape(a8, ref, dev, b, S):
    """The chooser's grid for the configs' row counts / cache lengths (C1, C2, C5's two passes, odd sizes)."""
    say(f"case: flat decode default shape b={b} S={S}")
    g = torch.Generator().manual_seed(34)
    q = randn_bf16(g, b, NQ, HD)
    kc, vc = randn_bf16(g, b, NKV, S, HD), randn_bf16(g, b, NKV, S, HD)
    lens = torch.randint(1, S + 1, (b,), generator=g).int()
    want = ref.decode_attention(q, kc, vc, lens)
    att = a8.DecodeAttention(max(16 * b, 8192) if S > 10 else max(2 * b, 16), NQ, NKV, HD, 16, dev)
    att.mode = "flat"
    kind, shape = att.schedule(b, S)
    say(f"  {kind} {shape}")
    assert kind == "flat"
    out = torch.empty(b, NQ, HD, dtype=BF, device=dev)
    att(q.to(dev), kc.to(dev), vc.to(dev), lens.to(dev), out)
    torch.cuda.synchronize()
    assert maxabs(out, want) <= TOL


def _store_inputs(seed, b, rows, S, lens, pos, slot, bias=True):
    g = torch.Generator().manual_seed(seed)
    return dict(qkv=randn_bf16(g, b, W), bias=(torch.randn(W, generator=g) * 0.02).to(BF) if bias else None,
                kc=randn_bf16(g, rows, NKV, S, HD), vc=randn_bf16(g, rows, NKV, S, HD),
                lens=torch.tensor(lens, dtype=torch.int32), pos=torch.tensor(pos, dtype=torch.int32),
                slot=torch.tensor(slot, dtype=torch.int32))


def _fused_vs_two_calls(a8, dev, x, grid, use_rowmap, ring=1 << 30, write_q=True):
    cos, sin = a8.rope_tables(10000.0, HD, 4096, dev)
    d = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in x.items()}
    b = d["qkv"].shape[0]
    att = a8.DecodeAttention(max(16 * b, 4096), NQ, NKV, HD, 16, dev)
    att.force_flat = grid
    rowmap = d["slot"] if use_rowmap else None
    res = []
    for fused in (False, True):
        kc, vc = d["kc"].clone(), d["vc"].clone()
        q = torch.zeros(b, NQ, HD, dtype=BF, device=dev)
        out = torch.empty(b, NQ, HD, dtype=BF, device=dev)
        if fused:
            att.store_and_attend(d["qkv"], d["bias"], cos, sin, d["pos"], d["slot"], q, kc, vc, d["lens"], out,
                                 rowmap=rowmap, ring=ring, write_q=write_q)
        else:
            a8.bias_rope_store(d["qkv"], d["bias"], cos, sin, d["pos"], d["slot"], q, kc, vc, NQ, NKV, HD, ring=ring)
            att(q, kc, vc, d["lens"], out, rowmap=rowmap)
        torch.cuda.synchronize()
        assert int(att.counters.abs().sum()) == 0
        res.append((out.cpu(), q.cpu(), kc.cpu(), vc.cpu()))
    return res


@pytest.mark.parametrize("grid", [1, 3, 16, 64])
def test_flat_fused_matches_two_calls(a8, dev, grid):
    """Store + decode in one flat launch equals bias_rope_store then the flat decode, bit for bit: ragged
    lengths, the new key at the end / inside / past the attended range, ring wrap, an invalid slot (NaN row,
    nothing stored), no bias; with rowmap = slot, and with no row map (row r attends cache row r; rows
    storing into their own row, a row past the query rows, or outside the cache)."""
    say(f"case: flat fused store+decode grid={grid}")
    S, rows, ring = 1024, 40, 1000
    lens = [1, 2, 64, 65, 1000, 700, 512, 1000, 300, 5, 900, 1000, 640, 1, 128, 999]
    pos = [0, 1, 63, 64, 999, 100, 900, 1500, 299, 4, 2, 1999, 639, 0, 127, 998]
    slot = [3, 7, 0, 39, 12, 5, 21, 9, 33, 2, 17, 28, 40, 11, 30, 1]   # slot 40: outside the cache
    b = len(lens)
    for bias in (True, False):
        x = _store_inputs(51 + bias, b, rows, S, lens, pos, slot, bias=bias)
        (o0, q0, k0, v0), (o1, q1, k1, v1) = _fused_vs_two_calls(a8, dev, x, grid, True, ring=ring)
        assert torch.equal(bits(q0), bits(q1))
        assert torch.equal(bits(k0), bits(k1)) and torch.equal(bits(v0), bits(v1))
        assert torch.equal(bits(o0), bits(o1))
        assert torch.isnan(o1[12].float()).all()
    slot2 = [r if r % 2 == 0 else (b + r if r % 4 == 1 else rows + 3) for r in range(b)]
    x = _store_inputs(53, b, rows, S, lens, pos, slot2)
    for write_q in (True, False):
        (o0, q0, k0, v0), (o1, q1, k1, v1) = _fused_vs_two_calls(a8, dev, x, grid, False, ring=ring, write_q=write_q)
        assert torch.equal(bits(q0), bits(q1)) if write_q else not q1.any()
        assert torch.equal(bits(k0), bits(k1)) and torch.equal(bits(v0), bits(v1))
        assert torch.equal(bits(o0), bits(o1))


def test_flat_graph_replays(a8, ref, dev):
    """A flat decode captured in a HIP graph: every replay (with eager work and new lengths between them)
    matches the eager call bit for bit, and the counters stay at zero."""
    say("case: flat decode graph replays")
    b, rows, S = 64, 64, 2048
    g, q, kc, vc, lens = _ragged(35, b, rows, S)
    att = a8.DecodeAttention(8192, NQ, NKV, HD, 16, dev)
    att.mode = "flat"
    qd, kd, vd, ld = q.to(dev), kc.to(dev), vc.to(dev), lens.to(dev)
    out = torch.empty(b, NQ, HD, dtype=BF, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            att(qd, kd, vd, ld, out)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        att(qd, kd, vd, ld, out)
    for rep in range(3):
        new = torch.randint(1, S + 1, (b,), generator=g).int()
        ld.copy_(new)
        graph.replay()
        torch.cuda.synchronize()
        got = out.cpu()
        eager = torch.empty_like(out)
        att(qd, kd, vd, ld, eager)
        torch.cuda.synchronize()
        assert torch.equal(bits(got), bits(eager.cpu())), rep
        assert int(att.counters.abs().sum()) == 0
        assert maxabs(got, ref.decode_attention(q, kc, vc, new)) <= TOL
