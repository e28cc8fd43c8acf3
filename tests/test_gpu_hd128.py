"""head_dim 128 (the reference kernels take HD as a compile-time constant, serve/fast_kernels.py:142, 196, 299;
the codec and fast-AR stacks get their head widths from the checkpoint, fast_engine.py:337, 608): the store
bit for bit against the oracle, decode at every benchmark config's shape through each schedule the package
can pick (split, stream, flat, the no-allocation entry and store_and_attend's two calls), packed prefill with
ragged requests and padding blocks, and the prefix copy. The oracle at 128 is pinned by the closed-form and
float64 textbook tests of test_oracle.py. Bar: max-abs <= 2e-2 (bit-exact for the store and the copy)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import randn_bf16

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
HD = 128
TOL = 2e-2


def say(msg):
    print(msg, flush=True)


def maxabs(a, b):
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


@pytest.mark.parametrize("nq,nkv,R,rows,S,ring", [(14, 2, 192, 193, 2048, 1 << 30), (8, 2, 37, 40, 300, 1 << 30),
                                                  (16, 4, 64, 16, 160, 128)])
def test_store_hd128(a8, ref, dev, nq, nkv, R, rows, S, ring):
    say(f"case: store hd 128 nq={nq} nkv={nkv} R={R} S={S} ring={ring}")
    g = torch.Generator().manual_seed(50 + nq)
    W = (nq + 2 * nkv) * HD
    qkv, bias = randn_bf16(g, R, W), randn_bf16(g, W, std=0.02)
    cos, sin = ref.rope_tables(10000.0, HD, 4 * S)
    # distinct (slot, position % ring) targets, so no two rows write one cache row
    span = min(ring, S)
    cell = torch.randperm(rows * span, generator=g)[:R]
    slot = (cell // span).int()
    pos = (cell % span + (ring * torch.randint(0, 3, (R,), generator=g) if ring < S else 0)).int()
    kc0, vc0 = randn_bf16(g, rows, nkv, S, HD), randn_bf16(g, rows, nkv, S, HD)
    qo_c = torch.zeros(R, nq, HD, dtype=BF)
    kc_c, vc_c = kc0.clone(), vc0.clone()
    ref.bias_rope_store(qkv, bias, cos, sin, pos, slot, qo_c, kc_c, vc_c, nq, nkv, HD, ring=ring)
    qo_d = torch.zeros(R, nq, HD, dtype=BF, device=dev)
    kc_d, vc_d = kc0.to(dev), vc0.to(dev)
    a8.bias_rope_store(qkv.to(dev), bias.to(dev), cos.to(dev), sin.to(dev), pos.to(dev), slot.to(dev), qo_d, kc_d,
                       vc_d, nq, nkv, HD, ring=ring)
    torch.cuda.synchronize()
    for got, want, name in ((qo_d, qo_c, "qo"), (kc_d, kc_c, "kc"), (vc_d, vc_c, "vc")):
        assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16)), name


def _decode_case(name, g, nq=14, nkv=2):
    if name == "C1":
        b, rows, S, lens = 1, 1, 512, torch.tensor([385])
    elif name == "C2":
        b, rows, S = 64, 65, 4096
        lens = torch.randint(128, 2049, (b,), generator=g)
    elif name == "C3":
        b, rows, S, lens = 192, 193, 2048, torch.full((192,), 2048)
    elif name == "C5a":
        b, rows, S, lens = 384, 192, 10, torch.arange(384) % 2 + 1
    else:  # edges: lens 0 (NaN like the reference), 1, tile multiples, > S (attends S)
        b, rows, S = 8, 8, 200
        lens = torch.tensor([0, 1, 63, 64, 65, 128, 200, 999])
    q = randn_bf16(g, b, nq, HD)
    kc, vc = randn_bf16(g, rows, nkv, S, HD), randn_bf16(g, rows, nkv, S, HD)
    rowmap = (torch.arange(b) // 2).int() if name == "C5a" else None
    return q, kc, vc, lens.int(), rowmap


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C5a", "edges"])
@pytest.mark.parametrize("mode", ["split", "stream", "flat"])
def test_decode_hd128(a8, ref, dev, name, mode):
    g = torch.Generator().manual_seed(61)
    q, kc, vc, lens, rowmap = _decode_case(name, g)
    b, S = q.shape[0], kc.shape[2]
    say(f"case: decode hd 128 {name} mode={mode} b={b} S={S}")
    want = ref.decode_attention(q, kc, vc, lens.clamp(max=S), nsplit=1, rowmap=rowmap)
    att = a8.DecodeAttention(max(16 * b, 64), 14, 2, HD, 16, dev)
    att.mode = mode
    out = torch.full((b, 14, HD), 3.0, dtype=BF, device=dev)
    att(q.to(dev), kc.to(dev), vc.to(dev), lens.to(dev), out, nsplit=4,
        rowmap=None if rowmap is None else rowmap.to(dev))
    torch.cuda.synchronize()
    got = out.cpu()
    nan_rows = (lens == 0).nonzero().flatten().tolist()
    for r in nan_rows:  # 0 / 0 like the reference
        assert torch.isnan(got[r].float()).all() and torch.isnan(want[r].float()).all()
    keep = [r for r in range(b) if r not in nan_rows]
    err = maxabs(got[keep], want[keep])
    say(f"  max-abs {err:.3e}")
    assert err <= TOL


def test_decode_hd128_noalloc_and_fused(a8, ref, dev):
    """The no-allocation entry point and store_and_attend (the store, then the decode) at head_dim 128."""
    say("case: decode hd 128 noalloc + store_and_attend")
    from audio8_turbo_engine_amd import _lib
    g = torch.Generator().manual_seed(62)
    nq, nkv, b, S = 14, 2, 48, 640
    q = randn_bf16(g, b, nq, HD)
    kc, vc = randn_bf16(g, b, nkv, S, HD), randn_bf16(g, b, nkv, S, HD)
    lens = torch.randint(1, S + 1, (b,), generator=g).int()
    want = ref.decode_attention(q, kc, vc, lens, nsplit=1)
    qd, kd, vd, ld = q.to(dev), kc.to(dev), vc.to(dev), lens.to(dev)
    out = torch.empty(b, nq, HD, dtype=BF, device=dev)
    st = _lib.load().a8_decode_attn_noalloc(qd.data_ptr(), qd.stride(0), qd.stride(1), kd.data_ptr(), vd.data_ptr(),
                                            kd.stride(0), kd.stride(1), kd.stride(2), kd.shape[0], S, ld.data_ptr(),
                                            None, out.data_ptr(), out.stride(0), out.stride(1), b, nq, nkv, HD, 4, 2,
                                            ctypes.c_float(HD ** -0.5), _lib.stream_of(qd))
    _lib.check(st, "decode_attn_noalloc")
    torch.cuda.synchronize()
    assert maxabs(out, want) <= TOL
    # store_and_attend == bias_rope_store then decode (and both match the oracle)
    W = (nq + 2 * nkv) * HD
    qkv, bias = randn_bf16(g, b, W), randn_bf16(g, W, std=0.02)
    cos, sin = ref.rope_tables(10000.0, HD, S)
    pos = (lens - 1).int()
    slot = torch.arange(b, dtype=torch.int32)
    kc_c, vc_c, q_c = kc.clone(), vc.clone(), torch.empty(b, nq, HD, dtype=BF)
    ref.bias_rope_store(qkv, bias, cos, sin, pos, slot, q_c, kc_c, vc_c, nq, nkv, HD)
    want = ref.decode_attention(q_c, kc_c, vc_c, lens, nsplit=1)
    att = a8.DecodeAttention(16 * b, nq, nkv, HD, 16, dev)
    kd2, vd2, qd2 = kc.to(dev), vc.to(dev), torch.empty(b, nq, HD, dtype=BF, device=dev)
    out2 = torch.empty(b, nq, HD, dtype=BF, device=dev)
    att.store_and_attend(qkv.to(dev), bias.to(dev), cos.to(dev), sin.to(dev), pos.to(dev), slot.to(dev), qd2, kd2,
                         vd2, ld, out2)
    torch.cuda.synchronize()
    assert torch.equal(kd2.cpu(), kc_c) and torch.equal(vd2.cpu(), vc_c) and torch.equal(qd2.cpu(), q_c)
    assert maxabs(out2, want) <= TOL


@pytest.mark.parametrize("nq,nkv", [(14, 2), (8, 8), (16, 1), (10, 2), (12, 2), (4, 4), (6, 2)])
def test_prefill_hd128(a8, ref, dev, nq, nkv):
    """Ragged requests after a prefix (one-tile to several-tile blocks, both halves of a block or only the first),
    with a padding block (n = 0), at every workgroup shape (q heads per kv head 7 -> 4 + 3, 1, 16 -> 4 x 4,
    5 -> 4 + 1, 6 -> 4 + 2, 3)."""
    group = nq // nkv
    say(f"case: prefill hd 128 nq={nq} nkv={nkv}")
    g = torch.Generator().manual_seed(70 + nq + nkv)
    S = 704
    ns = torch.randint(1, 300, (24,), generator=g).tolist()
    p0s = torch.randint(0, 300, (24,), generator=g).tolist()
    slots = torch.randperm(24, generator=g).tolist()
    r0s = [int(x) for x in np.cumsum([0] + ns[:-1])]
    R = sum(ns)
    kc, vc = randn_bf16(g, 25, nkv, S, HD), randn_bf16(g, 25, nkv, S, HD)
    q = randn_bf16(g, R, nq, HD)
    want = torch.zeros(R, nq, HD, dtype=BF)
    ref.prefill_attention(q, kc, vc, *ref.prefill_plan(r0s, ns, slots, p0s), want, group)
    plan = a8.PrefillPlan(r0s, ns, slots, p0s, dev)
    cols = [t.cpu().tolist() for t in (plan.q0, plan.n, plan.slot, plan.pos0)]
    blocks = list(zip(*cols)) + [(0, 0, 24, 0)]
    t = torch.tensor(blocks, dtype=torch.int32).T.contiguous().to(dev)

    class Plan:
        BM, nblk = 64, len(blocks)
        q0, n, slot, pos0 = t[0], t[1], t[2], t[3]

    out = torch.full((R, nq, HD), float("nan"), dtype=BF, device=dev)
    a8.prefill_attention(q.to(dev), kc.to(dev), vc.to(dev), Plan, out, group)
    torch.cuda.synchronize()
    err = maxabs(out, want)
    say(f"  R={R} blocks={len(blocks)} max-abs {err:.3e}")
    assert torch.isfinite(out.cpu().float()).all()
    assert err <= TOL


@pytest.mark.parametrize("first,later", [(-4.5, 1.0), (4.5, -4.5), (-2.0, 3.0)])
def test_prefill_hd128_extreme_scores(a8, ref, dev, first, later):
    """Scores far from 0 in exp2 units (q . k x scale x log2 e up to about +-200 at 128 dims): keys 0..31 (the
    first tile) `first` x ones, later keys `later` x ones, queries 3 x ones, plus noise. Covers the running
    offset's underflow guard, the raise on the first tile and a first tile far above the rest."""
    say(f"case: prefill hd 128 extreme scores, first tile {first}, later keys {later}")
    g = torch.Generator().manual_seed(int(first * 10 + later * 100) & 0xffff)
    nq, nkv = 14, 2
    ns, p0s, slots = [64, 150, 40, 1, 33], [100, 0, 400, 511, 31], [0, 1, 2, 3, 4]
    S, rows = 512, 5
    R = sum(ns)
    r0s = [int(x) for x in np.cumsum([0] + ns[:-1])]
    noise = lambda *shape: (torch.randn(*shape, generator=g) * 0.05)
    kc = torch.full((rows, nkv, S, HD), later) + noise(rows, nkv, S, HD)
    kc[:, :, :32] = first + noise(rows, nkv, 32, HD)
    kc = kc.to(BF)
    vc = randn_bf16(g, rows, nkv, S, HD)
    q = (3.0 + noise(R, nq, HD)).to(BF)
    want = torch.zeros(R, nq, HD, dtype=BF)
    ref.prefill_attention(q, kc, vc, *ref.prefill_plan(r0s, ns, slots, p0s), want, nq // nkv)
    out = torch.full((R, nq, HD), float("nan"), dtype=BF, device=dev)
    a8.prefill_attention(q.to(dev), kc.to(dev), vc.to(dev), a8.PrefillPlan(r0s, ns, slots, p0s, dev), out, nq // nkv)
    torch.cuda.synchronize()
    got = out.cpu()
    assert torch.isfinite(got.float()).all()
    err = maxabs(got, want)
    say(f"  max-abs {err:.3e}")
    assert err <= TOL


def test_attn_stack_prefill_hd128_fuse(a8, dev):
    """AttnStack at head_dim 128 with a prefill plan: fuse=True (no q-forming prefill at this width: the store
    writes q and the prefill reads it) gives the fuse=False bits."""
    say("case: stack prefill hd 128, fuse=True vs fuse=False")
    g = torch.Generator().manual_seed(77)
    nq, nkv, layers, rows, S = 14, 2, 2, 4, 512
    ns, p0s, slots = [100, 37, 64], [0, 200, 300], [2, 0, 1]
    R = sum(ns)
    W = (nq + 2 * nkv) * HD
    st = a8.AttnStack(layers, nq, nkv, HD, 10000.0, max_rows=R, cache_rows=rows, cache_len=S, max_pos=S, dev=dev)
    qkv = [randn_bf16(g, R, W).to(dev) for _ in range(layers)]
    bias = [randn_bf16(g, W, std=0.02).to(dev) for _ in range(layers)]
    pos = torch.cat([a + torch.arange(n) for a, n in zip(p0s, ns)]).int().to(dev)
    slot = torch.cat([torch.full((n,), s_) for s_, n in zip(slots, ns)]).int().to(dev)
    r0s = [int(x) for x in np.cumsum([0] + ns[:-1])]
    plan = a8.PrefillPlan(r0s, ns, slots, p0s, dev)
    kc0, vc0 = randn_bf16(g, layers, rows, nkv, S, HD).to(dev), randn_bf16(g, layers, rows, nkv, S, HD).to(dev)
    res = []
    for fuse in (False, True):
        st.kc_all.copy_(kc0)
        st.vc_all.copy_(vc0)
        q = torch.zeros(R, nq, HD, dtype=BF, device=dev)
        outs = [torch.zeros(R, nq, HD, dtype=BF, device=dev) for _ in range(layers)]
        st.forward(qkv, bias, pos, slot, None, plan=plan, q=q, outs=outs, fuse=fuse)
        torch.cuda.synchronize()
        res.append(([o.cpu() for o in outs], st.kc_all.cpu(), st.vc_all.cpu()))
    (o1, k1, v1), (o2, k2, v2) = res
    assert all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(o1, o2))
    assert torch.equal(k1.view(torch.int16), k2.view(torch.int16)) and torch.equal(v1.view(torch.int16), v2.view(torch.int16))
    assert all(torch.isfinite(o.float()).all() for o in o2)


def test_prefix_copy_hd128(a8, dev):
    say("case: prefix copy hd 128")
    g = torch.Generator().manual_seed(80)
    layers, rows, nkv, S, Lp = 3, 9, 2, 400, 300
    kc_all = randn_bf16(g, layers, rows, nkv, S, HD).to(dev)
    vc_all = randn_bf16(g, layers, rows, nkv, S, HD).to(dev)
    k, v = randn_bf16(g, layers, nkv, Lp, HD).to(dev), randn_bf16(g, layers, nkv, Lp, HD).to(dev)
    idx = [7, 2, 4]
    want_k, want_v = kc_all.clone(), vc_all.clone()
    want_k[:, idx, :, :Lp] = k.unsqueeze(1)
    want_v[:, idx, :, :Lp] = v.unsqueeze(1)
    a8.prefix_copy(k, v, kc_all, vc_all, idx)
    torch.cuda.synchronize()
    assert torch.equal(kc_all, want_k) and torch.equal(vc_all, want_v)
