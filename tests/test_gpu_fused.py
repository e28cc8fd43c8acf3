"""The fused store + decode launch (a8_store_decode_stream, DecodeAttention.store_and_attend) against the two
calls it replaces (bias_rope_store, then DecodeAttention, fast_engine.py:127-132) at the same streaming launch
shape: outputs, q and both caches bit for bit. Both row maps the engine uses: rowmap = slot (distinct slots)
and rowmap off (the decode tick, fast_engine.py:752-753: row r attends cache row r; here also rows that store
into a cache row no query row attends)."""
from __future__ import annotations

import pytest
import torch

from conftest import randn_bf16

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)

NQ, NKV, HD = 14, 2, 64
W = (NQ + 2 * NKV) * HD
BF = torch.bfloat16


def _inputs(seed, b, rows, S, lens, pos, slot, bias=True, max_pos=4096):
    g = torch.Generator().manual_seed(seed)
    qkv = randn_bf16(g, b, W)
    bb = (torch.randn(W, generator=g) * 0.02).to(BF) if bias else None
    kc, vc = randn_bf16(g, rows, NKV, S, HD), randn_bf16(g, rows, NKV, S, HD)
    return dict(qkv=qkv, bias=bb, kc=kc, vc=vc, lens=torch.tensor(lens, dtype=torch.int32),
                pos=torch.tensor(pos, dtype=torch.int32), slot=torch.tensor(slot, dtype=torch.int32),
                max_pos=max_pos)


def _run_both(a8, dev, x, shape, ring=1 << 30, write_q=True, use_rowmap=True, split=False, merge=False):
    cos, sin = a8.rope_tables(10000.0, HD, x["max_pos"], dev)
    b = x["qkv"].shape[0]
    d = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in x.items()}
    att = a8.DecodeAttention(max(16 * b, 8192), NQ, NKV, HD, 16, dev)
    att.merge_in_kernel = merge
    if split:
        att.force_shape = shape   # (nsplit, waves): the split + combine schedule, store in the split kernel
    else:
        att.force_stream = shape
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
        res.append((out.cpu(), q.cpu(), kc.cpu(), vc.cpu()))
    return res


def _bits_equal(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("shape", [(4, 8, 48), (4, 8, 192)])
@pytest.mark.parametrize("mode", ["rowmap=slot", "tick", "rowmap off, mixed slots"])
def test_store_and_attend_peak_shape(a8, dev, mode, shape):
    """The C3 launch shape (whole 2048-key rows, 4 waves, 2 units per workgroup) and the one-unit-per-workgroup
    launch, rows at pos = lens - 1: shuffled slots attended through the row map; the tick (slot = row, no row
    map); no row map with some rows storing into their own cache row and others into rows past the query rows
    (no new key seen)."""
    say(f"case: fused store+decode, 96 rows x 2048, shape {shape}, {mode}")
    b, S = 96, 2048
    g = torch.Generator().manual_seed(41)
    if mode == "rowmap=slot":
        slot = torch.randperm(b + 4, generator=g)[:b].tolist()
    elif mode == "tick":
        slot = list(range(b))
    else:
        slot = [r if r % 3 else b + r // 3 for r in range(b)]
    lens = [S] * (b - 8) + [1, 2, 63, 64, 65, 1000, 2047, 129]
    pos = [L - 1 for L in lens]
    x = _inputs(41, b, max(slot) + 1, S, lens, pos, slot)
    for write_q in (True, False):
        (o0, q0, k0, v0), (o1, q1, k1, v1) = _run_both(a8, dev, x, shape, write_q=write_q,
                                                       use_rowmap=(mode == "rowmap=slot"))
        assert _bits_equal(q0, q1) if write_q else not q1.any()           # q untouched when not asked for
        assert _bits_equal(k0, k1) and _bits_equal(v0, v1)
        assert _bits_equal(o0, o1)
        assert not torch.isnan(o1.float()).any()


@pytest.mark.parametrize("shape", [(4, 8, 64), (4, 2, 100), (2, 2, 37), (1, 2, 9), (1, 1, 200), (2, 16, 5),
                                   (4, 4, 1), (4, 4, 16), (4, 4, 32)])
def test_store_and_attend_edge_rows(a8, dev, shape):
    """Ragged lengths; the new key at the end, in the middle of the attended range (lens > pos + 1) or past
    it (pos >= lens); ring wrap (pos >= ring); a slot outside the cache (NaN row, nothing stored); no
    bias; chunks shorter than a row (merge kernel) and 128-key steps."""
    say(f"case: fused store+decode edge rows, shape {shape}")
    S, rows, ring = 1024, 40, 1000
    lens = [1, 2, 64, 65, 1000, 700, 512, 1000, 300, 5, 900, 1000, 640, 1, 128, 999]
    pos = [0, 1, 63, 64, 999, 100, 900, 1500, 299, 4, 2, 1999, 639, 0, 127, 998]
    slot = [3, 7, 0, 39, 12, 5, 21, 9, 33, 2, 17, 28, 40, 11, 30, 1]   # slot 40: outside the cache
    b = len(lens)
    for bias in (True, False):
        x = _inputs(43 + bias, b, rows, S, lens, pos, slot, bias=bias)
        (o0, q0, k0, v0), (o1, q1, k1, v1) = _run_both(a8, dev, x, shape, ring=ring)
        assert _bits_equal(q0, q1)
        assert _bits_equal(k0, k1) and _bits_equal(v0, v1)
        assert _bits_equal(o0, o1)
        assert torch.isnan(o1[12].float()).all()                       # slot 40 does not exist
    # no row map: row r attends cache row r; rows store into their own row, rows >= b or outside the cache
    slot2 = [r if r % 2 == 0 else (b + r if r % 4 == 1 else rows + 3) for r in range(b)]
    x = _inputs(45, b, rows, S, lens, pos, slot2)
    (o0, q0, k0, v0), (o1, q1, k1, v1) = _run_both(a8, dev, x, shape, ring=ring, use_rowmap=False)
    assert _bits_equal(q0, q1)
    assert _bits_equal(k0, k1) and _bits_equal(v0, v1)
    assert _bits_equal(o0, o1)


def test_store_and_attend_positions_outside_tables(a8, dev):
    """A row whose position is outside the RoPE tables stores nothing (like the store kernel); the other
    rows are unaffected and identical to the two calls."""
    say("case: fused store+decode, positions outside the tables")
    S, rows = 512, 8
    lens, pos, slot = [100, 200, 300, 512], [99, 5000, -3, 511], [0, 1, 2, 3]
    x = _inputs(47, 4, rows, S, lens, pos, slot, max_pos=1024)
    (o0, q0, k0, v0), (o1, q1, k1, v1) = _run_both(a8, dev, x, (4, 2, 8))
    assert _bits_equal(k0, k1) and _bits_equal(v0, v1)
    for r in (0, 3):
        assert _bits_equal(o0[r], o1[r]) and _bits_equal(q0[r], q1[r])
    assert torch.isfinite(o1[1:3].float()).all()                       # q = 0: the mean of the values


def test_attn_stack_tick_fused_matches_unfused(a8, dev):
    """AttnStack.forward (the engine's per-layer order) with the fused launch equals the two-call path for
    a 3-layer stack, caches included, at the peak-load schedule."""
    say("case: 3-layer stack, fused vs unfused tick")
    b, S, L = 64, 2048, 3
    st = [a8.AttnStack(L, NQ, NKV, HD, 10000.0, max_rows=8192, cache_rows=b, cache_len=S, max_pos=S, dev=dev)
          for _ in range(2)]
    g = torch.Generator(device=dev).manual_seed(5)
    for i in range(L):
        st[0].kc[i].normal_(generator=g)
        st[0].vc[i].normal_(generator=g)
        st[1].kc[i].copy_(st[0].kc[i])
        st[1].vc[i].copy_(st[0].vc[i])
    lens = torch.full((b,), S, dtype=torch.int32, device=dev)
    lens[:5] = torch.tensor([1, 700, 1500, 2000, 64], dtype=torch.int32)
    pos, slot = lens - 1, torch.arange(b, dtype=torch.int32, device=dev)
    qkv = [torch.randn(b, W, generator=g, device=dev).to(BF) for _ in range(L)]
    bias = [(torch.randn(W, generator=g, device=dev) * 0.02).to(BF) for _ in range(L)]
    outs = []
    for k, fuse in enumerate((False, True)):
        st[k].attn.force_stream = (4, 8, 32)
        outs.append(st[k].forward(qkv, bias, pos, slot, lens, rowmap=False, fuse=fuse))
    torch.cuda.synchronize()
    for i in range(L):
        assert _bits_equal(outs[0][i], outs[1][i])
        assert _bits_equal(st[0].kc[i], st[1].kc[i]) and _bits_equal(st[0].vc[i], st[1].vc[i])


@pytest.mark.parametrize("b,S", [(1, 512), (192, 10), (64, 300), (5, 65)])
def test_store_and_attend_short_rows_auto(a8, ref, dev, b, S):
    """Mode "auto" runs a fused call over short rows (cache_len <= 512) as one streaming launch with one
    workgroup per (row, kv head): the same bits as the two calls at that launch shape, and the oracle's
    answer (the engine's tick: slot = row, no row map)."""
    say(f"case: fused short rows auto, b={b} S={S}")
    g = torch.Generator().manual_seed(61)
    lens = torch.randint(1, S + 1, (b,), generator=g).tolist()
    pos = [L - 1 for L in lens]
    x = _inputs(61, b, b, S, lens, pos, list(range(b)), max_pos=S)
    att = a8.DecodeAttention(max(16 * b, 64), NQ, NKV, HD, 16, dev)
    kind, shape = att.schedule(b, S, fused=True)
    assert kind == "stream" and shape[2] == 2 * b and shape[0] * shape[1] * 64 >= S
    (o0, q0, k0, v0), (o1, q1, k1, v1) = _run_both(a8, dev, x, shape, use_rowmap=False)
    assert _bits_equal(k0, k1) and _bits_equal(v0, v1) and _bits_equal(q0, q1)
    assert _bits_equal(o0, o1)
    want = ref.decode_attention(q0, k0, v0, torch.tensor(lens, dtype=torch.int32))
    assert (o1.float() - want.float()).abs().max().item() <= 2e-2


@pytest.mark.parametrize("shape,merge", [((1, 1), False), ((1, 4), False), ((3, 2), False), ((4, 1), False),
                                         ((8, 4), False), ((16, 1), False), ((3, 2), True), ((4, 1), True),
                                         ((16, 1), True)])
def test_store_and_attend_split_schedule(a8, dev, shape, merge):
    """The store done by the split kernel (a8_store_decode_split) equals bias_rope_store then the split
    decode at the same (nsplit, waves), bit for bit: the edge rows of the streaming test (new key at the end,
    inside or past the attended range, ring wrap, a slot outside the cache, no bias), with rowmap = slot and
    with no row map; also with the splits merged inside the split kernel (merge)."""
    say(f"case: fused store + split decode, shape {shape}, merge in kernel {merge}")
    S, rows, ring = 1024, 40, 1000
    lens = [1, 2, 64, 65, 1000, 700, 512, 1000, 300, 5, 900, 1000, 640, 1, 128, 999]
    pos = [0, 1, 63, 64, 999, 100, 900, 1500, 299, 4, 2, 1999, 639, 0, 127, 998]
    slot = [3, 7, 0, 39, 12, 5, 21, 9, 33, 2, 17, 28, 40, 11, 30, 1]
    b = len(lens)
    for bias in (True, False):
        x = _inputs(71 + bias, b, rows, S, lens, pos, slot, bias=bias)
        (o0, q0, k0, v0), (o1, q1, k1, v1) = _run_both(a8, dev, x, shape, ring=ring, split=True, merge=merge)
        assert _bits_equal(q0, q1)
        assert _bits_equal(k0, k1) and _bits_equal(v0, v1)
        assert _bits_equal(o0, o1)
        assert torch.isnan(o1[12].float()).all()
    slot2 = [r if r % 2 == 0 else (b + r if r % 4 == 1 else rows + 3) for r in range(b)]
    x = _inputs(73, b, rows, S, lens, pos, slot2)
    for write_q in (True, False):
        (o0, q0, k0, v0), (o1, q1, k1, v1) = _run_both(a8, dev, x, shape, ring=ring, write_q=write_q,
                                                       use_rowmap=False, split=True, merge=merge)
        assert _bits_equal(q0, q1) if write_q else not q1.any()
        assert _bits_equal(k0, k1) and _bits_equal(v0, v1)
        assert _bits_equal(o0, o1)

