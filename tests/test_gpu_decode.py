"""GPU parity of split-K decode attention (DecodeAttention -> a8_decode_attn) against the golden vectors and
the CPU oracle at every benchmark config's shape (C1-C5), over launch shapes, row maps, strides and edge lengths.
Bar: max-abs <= 2e-2 on the bf16 outputs (fp32 softmax / accumulate, bf16 out)."""
from __future__ import annotations

import pytest
import torch

from conftest import bf16_from_bits, golden, randn_bf16

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
NQ, NKV, HD = 14, 2, 64
TOL = 2e-2


def say(msg):
    print(msg, flush=True)


def maxabs(a, b):
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


def run_gpu(a8, dev, q, kc, vc, lens, rowmap=None, nsplit=1, cap=None, nsplit_max=16, shape=None, kcv=None, vcv=None):
    b = q.shape[0]
    att = a8.DecodeAttention(cap or max(16 * b, 64), NQ, NKV, HD, nsplit_max, dev)
    att.force_shape = shape
    out = torch.empty(b, NQ, HD, dtype=BF, device=dev)
    att(q.to(dev), kc.to(dev) if kcv is None else kcv, vc.to(dev) if vcv is None else vcv, lens.to(dev), out,
        nsplit=nsplit, rowmap=None if rowmap is None else rowmap.to(dev))
    torch.cuda.synchronize()
    return out.cpu(), att


def test_decode_golden(a8, dev):
    z = golden("decode.npz")
    q, kc, vc = bf16_from_bits(z["q"]), bf16_from_bits(z["kc"]), bf16_from_bits(z["vc"])
    lens, rowmap = torch.from_numpy(z["lens"]), torch.from_numpy(z["rowmap"])
    want = torch.from_numpy(z["out"])
    for shape in (None, (1, 1), (1, 4), (3, 2), (5, 8)):
        say(f"case: decode golden shape={shape}")
        out, _ = run_gpu(a8, dev, q, kc, vc, lens, rowmap, shape=shape)
        assert maxabs(out, want) <= TOL, shape


def _cfg(name, g):
    """(q, kc, vc, lens, rowmap, nsplit_max) at a benchmark config's shape (one layer)."""
    if name == "C1":
        b, rows, S = 1, 1, 512
        lens = torch.tensor([385])
    elif name == "C2":
        b, rows, S = 64, 65, 4096
        lens = torch.randint(128, 2049, (b,), generator=g)
    elif name == "C3":
        b, rows, S = 192, 193, 2048
        lens = torch.full((b,), 2048)
    elif name == "C5a":
        b, rows, S = 384, 192, 10
        lens = torch.arange(b) % 2 + 1
    elif name == "C5b":
        b, rows, S = 192, 192, 10
        lens = torch.randint(3, 11, (b,), generator=g)
    q = randn_bf16(g, b, NQ, HD)
    kc, vc = randn_bf16(g, rows, NKV, S, HD), randn_bf16(g, rows, NKV, S, HD)
    rowmap = (torch.arange(b) // 2).int() if name == "C5a" else None
    return q, kc, vc, lens.int(), rowmap, (1 if name.startswith("C5") else 16)


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C5a", "C5b"])
def test_decode_configs(a8, ref, dev, name):
    g = torch.Generator().manual_seed(21)
    q, kc, vc, lens, rowmap, nmax = _cfg(name, g)
    say(f"case: decode {name} b={q.shape[0]} S={kc.shape[2]}")
    want = ref.decode_attention(q, kc, vc, lens, nsplit=1, rowmap=rowmap)
    out, att = run_gpu(a8, dev, q, kc, vc, lens, rowmap, nsplit=ref.ref_nsplit(q.shape[0], NKV), nsplit_max=nmax)
    err = maxabs(out, want)
    say(f"  launch shape {att.launch_shape(q.shape[0], kc.shape[2], 1)} max-abs {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("ns,nw", [(1, 1), (1, 2), (1, 8), (2, 4), (3, 1), (4, 8), (7, 2), (16, 4), (32, 1)])
def test_decode_launch_shapes(a8, ref, dev, ns, nw):
    """Every split count / waves-per-split gives the oracle's answer (ragged lengths incl. tile edges)."""
    say(f"case: decode launch shape nsplit={ns} waves={nw}")
    g = torch.Generator().manual_seed(22)
    b, S = 12, 1100
    q = randn_bf16(g, b, NQ, HD)
    kc, vc = randn_bf16(g, b, NKV, S, HD), randn_bf16(g, b, NKV, S, HD)
    lens = torch.tensor([1, 2, 63, 64, 65, 127, 128, 129, 500, 1023, 1100, 777], dtype=torch.int32)
    want = ref.decode_attention(q, kc, vc, lens, nsplit=1)
    out, _ = run_gpu(a8, dev, q, kc, vc, lens, shape=(ns, nw), cap=b * 32)
    assert maxabs(out, want) <= TOL


@pytest.mark.parametrize("ns,nw", [(2, 1), (4, 1), (16, 1), (3, 2), (4, 4), (9, 8)])
def test_decode_merge_in_kernel(a8, ref, dev, ns, nw):
    """The split kernel's own merge (last split to finish, arrival counters) gives the bits of the split +
    combine launches, leaves every counter at zero, and the next call (fewer rows) is right as well."""
    say(f"case: decode in-kernel merge nsplit={ns} waves={nw}")
    g = torch.Generator().manual_seed(26)
    b, S = 12, 1100
    q = randn_bf16(g, b, NQ, HD).to(dev)
    kc, vc = randn_bf16(g, b, NKV, S, HD).to(dev), randn_bf16(g, b, NKV, S, HD).to(dev)
    lens = torch.tensor([1, 2, 63, 64, 65, 127, 128, 129, 500, 1023, 1100, 0], dtype=torch.int32).to(dev)
    att = a8.DecodeAttention(b * 16, NQ, NKV, HD, 16, dev)
    att.force_shape = (ns, nw)
    outs = {}
    for merge in (False, True, True):
        att.merge_in_kernel = merge
        o = torch.full((b, NQ, HD), 7.0, dtype=BF, device=dev)
        att(q, kc, vc, lens, o)
        torch.cuda.synchronize()
        outs.setdefault(merge, []).append(o.cpu())
        assert int(att.counters.abs().sum()) == 0
    assert torch.equal(outs[True][0].view(torch.int16), outs[False][0].view(torch.int16))
    assert torch.equal(outs[True][1].view(torch.int16), outs[False][0].view(torch.int16))
    want = ref.decode_attention(q.cpu()[:11], kc.cpu()[:11], vc.cpu()[:11], lens.cpu()[:11], nsplit=1)
    assert maxabs(outs[True][0][:11], want) <= TOL
    assert torch.isnan(outs[True][0][11].float()).all()  # lens 0: 0/0 as the reference
    # a smaller call through the same counters and workspace
    o = torch.empty(5, NQ, HD, dtype=BF, device=dev)
    att(q[:5], kc, vc, lens[:5], o)
    torch.cuda.synchronize()
    assert torch.equal(o.cpu().view(torch.int16), outs[False][0][:5].view(torch.int16))
    assert int(att.counters.abs().sum()) == 0


def test_decode_edge_lengths(a8, dev):
    say("case: decode L=0 / L=1 / lens > S")
    g = torch.Generator().manual_seed(23)
    b, S = 4, 96
    q = randn_bf16(g, b, NQ, HD)
    kc, vc = randn_bf16(g, b, NKV, S, HD), randn_bf16(g, b, NKV, S, HD)
    for shape in ((1, 1), (1, 4), (3, 2)):
        out, _ = run_gpu(a8, dev, q, kc, vc, torch.tensor([0, 1, 1, 0], dtype=torch.int32), shape=shape)
        assert torch.isnan(out[0].float()).all() and torch.isnan(out[3].float()).all()      # 0/0 as the reference
        for i in (1, 2):                                                                     # the one value row
            assert torch.equal(out[i, :7], vc[i, 0, 0].expand(7, HD))
            assert torch.equal(out[i, 7:], vc[i, 1, 0].expand(7, HD))
    # lens past the cache are clamped to the cache length (the reference would read out of bounds)
    full, _ = run_gpu(a8, dev, q, kc, vc, torch.full((b,), S, dtype=torch.int32), shape=(2, 2))
    over, _ = run_gpu(a8, dev, q, kc, vc, torch.full((b,), S + 500, dtype=torch.int32), shape=(2, 2))
    assert torch.equal(full, over)


def test_decode_rowmap_and_strided_cache(a8, ref, dev):
    say("case: decode rowmap + arena-strided cache")
    g = torch.Generator().manual_seed(24)
    b, rows, S = 9, 5, 128
    q = randn_bf16(g, b, NQ, HD)
    kc, vc = randn_bf16(g, rows, NKV, S, HD), randn_bf16(g, rows, NKV, S, HD)
    lens = torch.randint(1, S + 1, (b,), generator=g).int()
    rowmap = torch.randint(0, rows, (b,), generator=g).int()
    want = ref.decode_attention(q, kc, vc, lens, rowmap=rowmap)
    per = NKV * S * HD
    buf = torch.zeros(rows, 2 * per + 40, dtype=BF, device=dev)
    kv = buf[:, 8:8 + per].view(rows, NKV, S, HD)
    vv = buf[:, per + 16:2 * per + 16].view(rows, NKV, S, HD)
    kv.copy_(kc.to(dev))
    vv.copy_(vc.to(dev))
    for shape in ((1, 2), (2, 1), (4, 4)):
        out, _ = run_gpu(a8, dev, q, kc, vc, lens, rowmap, shape=shape, kcv=kv, vcv=vv)
        assert maxabs(out, want) <= TOL


def test_decode_phases_split_then_combine(a8, ref, dev):
    """The split and combine kernels (and the streaming and merge kernels) launched one at a time give the
    same bits as one call."""
    say("case: decode phases 1 then 2")
    g = torch.Generator().manual_seed(25)
    b, S = 16, 700
    q = randn_bf16(g, b, NQ, HD).to(dev)
    kc, vc = randn_bf16(g, b, NKV, S, HD).to(dev), randn_bf16(g, b, NKV, S, HD).to(dev)
    lens = torch.randint(1, S + 1, (b,), generator=g).int().to(dev)
    att = a8.DecodeAttention(16 * b, NQ, NKV, HD, 16, dev)
    att.merge_in_kernel = False  # the split + combine launches (the in-kernel merge has one phase)
    for split, stream in (((5, 2), None), (None, (2, 1, 9))):
        att.force_shape, att.force_stream = split, stream
        o1, o2 = torch.empty(b, NQ, HD, dtype=BF, device=dev), torch.empty(b, NQ, HD, dtype=BF, device=dev)
        att(q, kc, vc, lens, o1)
        att(q, kc, vc, lens, o2, phases=1)
        att(q, kc, vc, lens, o2, phases=2)
        torch.cuda.synchronize()
        assert torch.equal(o1.cpu(), o2.cpu())


def test_decode_after_store_c1(a8, ref, dev):
    """Config 1 end to end: store the new token at 384, then attend 385 keys."""
    say("case: decode C1 store + attend")
    g = torch.Generator().manual_seed(26)
    W = (NQ + 2 * NKV) * HD
    qkv, bias = randn_bf16(g, 1, W), randn_bf16(g, W, std=0.02)
    kc, vc = randn_bf16(g, 1, NKV, 512, HD), randn_bf16(g, 1, NKV, 512, HD)
    cos, sin = ref.rope_tables(10000.0, HD, 2048)
    pos, slot = torch.tensor([384], dtype=torch.int32), torch.tensor([0], dtype=torch.int32)
    qc, kcc, vcc = torch.empty(1, NQ, HD, dtype=BF), kc.clone(), vc.clone()
    ref.bias_rope_store(qkv, bias, cos, sin, pos, slot, qc, kcc, vcc, NQ, NKV, HD)
    want = ref.decode_attention(qc, kcc, vcc, pos + 1)
    qd, kcd, vcd = torch.empty(1, NQ, HD, dtype=BF, device=dev), kc.to(dev), vc.to(dev)
    a8.bias_rope_store(qkv.to(dev), bias.to(dev), cos.to(dev), sin.to(dev), pos.to(dev), slot.to(dev), qd, kcd, vcd,
                       NQ, NKV, HD)
    out, _ = run_gpu(a8, dev, qd.cpu(), kcd.cpu(), vcd.cpu(), pos + 1)
    assert maxabs(out, want) <= TOL


@pytest.mark.parametrize("nw,tpw,grid", [(4, 2, 512), (4, 2, 1), (4, 2, 3), (1, 1, 7), (2, 1, 64), (2, 2, 256),
                                         (4, 4, 100), (1, 3, 1000), (1, 2, 2), (2, 8, 40), (4, 6, 40), (4, 8, 20)])
def test_decode_stream_shapes(a8, ref, dev, nw, tpw, grid):
    """The streaming kernel at forced launch shapes: chunks of nw * tpw * 64 keys swept by `grid`
    workgroups (grid 1: one workgroup takes every chunk; 64-key chunks: many partials per row, merged by
    the merge kernel; waves <= 2 with an even tile count: 128-key steps; whole rows at one unit per
    workgroup and at two: the unit and rows kernels, tiles past the cache length requested and dropped). Ragged
    lengths, a row map, empty rows; two calls in a row give the same bits."""
    say(f"case: decode stream waves={nw} tpw={tpw} grid={grid}")
    g = torch.Generator().manual_seed(27)
    b, rows, S = 20, 9, 1500
    q = randn_bf16(g, b, NQ, HD)
    kc, vc = randn_bf16(g, rows, NKV, S, HD), randn_bf16(g, rows, NKV, S, HD)
    lens = torch.randint(1, S + 1, (b,), generator=g).int()
    lens[:6] = torch.tensor([0, 1, 64, 65, 1500, 0], dtype=torch.int32)
    rowmap = torch.randint(0, rows, (b,), generator=g).int()
    want = ref.decode_attention(q, kc, vc, lens, rowmap=rowmap)
    att = a8.DecodeAttention(b * 32, NQ, NKV, HD, 16, dev)
    att.force_stream = (nw, tpw, grid)
    outs = []
    for _ in range(2):
        out = torch.empty(b, NQ, HD, dtype=BF, device=dev)
        att(q.to(dev), kc.to(dev), vc.to(dev), lens.to(dev), out, rowmap=rowmap.to(dev))
        torch.cuda.synchronize()
        outs.append(out.cpu())
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    o = outs[0]
    assert torch.isnan(o[0].float()).all() and torch.isnan(o[5].float()).all()
    assert maxabs(o[1:5], want[1:5]) <= TOL and maxabs(o[6:], want[6:]) <= TOL


def test_decode_stream_default_shapes_all_configs(a8, ref, dev):
    """The chooser's shape for each config's row count / cache length runs and matches the oracle."""
    g = torch.Generator().manual_seed(28)
    for b, S in ((1, 512), (64, 4096), (192, 2048), (384, 10), (7, 100), (300, 3000)):
        say(f"case: decode stream default shape b={b} S={S}")
        q = randn_bf16(g, b, NQ, HD)
        kc, vc = randn_bf16(g, b, NKV, S, HD), randn_bf16(g, b, NKV, S, HD)
        lens = torch.randint(1, S + 1, (b,), generator=g).int()
        want = ref.decode_attention(q, kc, vc, lens)
        out, att = run_gpu(a8, dev, q, kc, vc, lens, cap=max(16 * b, 8192))
        say(f"  shape {att.stream_shape(b, S)}")
        assert maxabs(out, want) <= TOL
