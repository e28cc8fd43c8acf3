"""GPU parity of packed causal prefill attention (prefill_attention -> a8_prefill_attn) against the golden
vectors and the CPU oracle, incl. config 4 at full size (voice-prefix KV copied into the slots, then
store + prefill) and the graph-mode plan with padding blocks. Bar: max-abs <= 2e-2."""
from __future__ import annotations

import numpy as np
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


def test_prefill_golden(a8, dev):
    say("case: prefill golden")
    z = golden("prefill.npz")
    q, kc, vc = bf16_from_bits(z["q"]), bf16_from_bits(z["kc"]), bf16_from_bits(z["vc"])
    reqs = z["reqs"]
    ns = [int(n) for _, _, n in reqs]
    r0s = [int(x) for x in np.cumsum([0] + ns[:-1])]
    plan = a8.PrefillPlan(r0s, ns, [int(s) for s, _, _ in reqs], [int(p) for _, p, _ in reqs], dev)
    out = torch.zeros_like(q, device=dev)
    a8.prefill_attention(q.to(dev), kc.to(dev), vc.to(dev), plan, out, 7)
    torch.cuda.synchronize()
    assert maxabs(out, torch.from_numpy(z["out"].astype(np.float32))) <= TOL


def _c4(g, n_req=64, lo=40, hi=400, p0=300, voices=4):
    ns = torch.randint(lo, hi + 1, (n_req,), generator=g).tolist()
    S = p0 + hi + 4
    prefix_k = [randn_bf16(g, NKV, p0, HD) for _ in range(voices)]
    prefix_v = [randn_bf16(g, NKV, p0, HD) for _ in range(voices)]
    return ns, S, prefix_k, prefix_v


def test_prefill_c4_full(a8, ref, dev):
    """Config 4: 64 requests, n ~ U[40, 400], each after a 300-position voice prefix (4 voices x 16 slots)."""
    say("case: prefill C4 full size")
    g = torch.Generator().manual_seed(31)
    ns, S, pk, pv = _c4(g)
    p0 = 300
    nreq = len(ns)
    rows = nreq + 1
    W = (NQ + 2 * NKV) * HD
    R = sum(ns)
    qkv, bias = randn_bf16(g, R, W), randn_bf16(g, W, std=0.02)
    cos, sin = ref.rope_tables(10000.0, HD, 2048)
    pos = torch.cat([p0 + torch.arange(n) for n in ns]).int()
    slot = torch.cat([torch.full((n,), i) for i, n in enumerate(ns)]).int()
    r0s = [int(x) for x in np.cumsum([0] + ns[:-1])]
    # host oracle: prefix copy (voice i % 4), store, prefill
    kc = torch.zeros(rows, NKV, S, HD, dtype=BF)
    vc = torch.zeros_like(kc)
    for i in range(nreq):
        kc[i, :, :p0], vc[i, :, :p0] = pk[i % 4], pv[i % 4]
    kcd, vcd = kc.to(dev), vc.to(dev)
    q_c = torch.empty(R, NQ, HD, dtype=BF)
    ref.bias_rope_store(qkv, bias, cos, sin, pos, slot, q_c, kc, vc, NQ, NKV, HD)
    out_c = torch.zeros(R, NQ, HD, dtype=BF)
    ref.prefill_attention(q_c, kc, vc, *ref.prefill_plan(r0s, ns, list(range(nreq)), [p0] * nreq), out_c, 7)
    # GPU
    q_d = torch.empty(R, NQ, HD, dtype=BF, device=dev)
    a8.bias_rope_store(qkv.to(dev), bias.to(dev), cos.to(dev), sin.to(dev), pos.to(dev), slot.to(dev), q_d, kcd, vcd,
                       NQ, NKV, HD)
    plan = a8.PrefillPlan(r0s, ns, list(range(nreq)), [p0] * nreq, dev)
    out_d = torch.zeros(R, NQ, HD, dtype=BF, device=dev)
    a8.prefill_attention(q_d, kcd, vcd, plan, out_d, 7)
    torch.cuda.synchronize()
    assert torch.equal(q_d.cpu(), q_c) and torch.equal(kcd.cpu(), kc) and torch.equal(vcd.cpu(), vc)
    err = maxabs(out_d, out_c)
    say(f"  R={R} blocks={plan.nblk} max-abs {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("seed", [0, 1])
def test_prefill_random_cache(a8, ref, dev, seed):
    """16 requests, n ~ U[40, 400], after a 300-position prefix, over a cache and queries drawn at random
    (no store first): every output row finite and within the bar of the oracle."""
    say(f"case: prefill random cache, seed {seed}")
    g = torch.Generator().manual_seed(100 + seed)
    ns = torch.randint(40, 401, (16,), generator=g).tolist()
    p0, S, nreq = 300, 704, 16
    R = sum(ns)
    kc, vc = randn_bf16(g, nreq + 1, NKV, S, HD), randn_bf16(g, nreq + 1, NKV, S, HD)
    q = randn_bf16(g, R, NQ, HD)
    r0s = [int(x) for x in np.cumsum([0] + ns[:-1])]
    want = torch.zeros(R, NQ, HD, dtype=BF)
    ref.prefill_attention(q, kc, vc, *ref.prefill_plan(r0s, ns, list(range(nreq)), [p0] * nreq), want, 7)
    out = torch.full((R, NQ, HD), float("nan"), dtype=BF, device=dev)
    a8.prefill_attention(q.to(dev), kc.to(dev), vc.to(dev), a8.PrefillPlan(r0s, ns, list(range(nreq)), [p0] * nreq, dev),
                         out, 7)
    torch.cuda.synchronize()
    got = out.cpu()
    assert torch.isfinite(got.float()).all()
    err = maxabs(got, want)
    say(f"  R={R} max-abs {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("first,later", [(-4.5, 1.0), (-4.5, -4.5), (4.5, 4.5), (4.5, -4.5), (-2.0, 3.0)])
def test_prefill_extreme_scores(a8, ref, dev, first, later):
    """Scores far from 0 in exp2 units (q . k x scale x log2 e up to about +-207): the keys of each block's first
    tile (positions 0..63) and the later keys are `first` and `later` times a ones vector (plus noise), the
    queries 4 x ones. Covers the running offset's underflow guard (every first-tile score far below 0,
    later ones higher or as low), the raise on the first tile (far above 0) and a first tile far above the
    rest; every row finite and within the bar of the oracle."""
    say(f"case: prefill extreme scores, first tile {first}, later keys {later}")
    g = torch.Generator().manual_seed(int(first * 10 + later * 100) & 0xffff)
    ns, p0s, slots = [64, 150, 40, 1], [100, 0, 400, 511], [0, 1, 2, 3]
    S, rows = 512, 4
    R = sum(ns)
    r0s = [int(x) for x in np.cumsum([0] + ns[:-1])]
    noise = lambda *shape: (torch.randn(*shape, generator=g) * 0.05)
    kc = (torch.full((rows, NKV, S, HD), later) + noise(rows, NKV, S, HD))
    kc[:, :, :64] = first + noise(rows, NKV, 64, HD)
    kc = kc.to(BF)
    vc = randn_bf16(g, rows, NKV, S, HD)
    q = (4.0 + noise(R, NQ, HD)).to(BF)
    want = torch.zeros(R, NQ, HD, dtype=BF)
    ref.prefill_attention(q, kc, vc, *ref.prefill_plan(r0s, ns, slots, p0s), want, 7)
    out = torch.full((R, NQ, HD), float("nan"), dtype=BF, device=dev)
    a8.prefill_attention(q.to(dev), kc.to(dev), vc.to(dev), a8.PrefillPlan(r0s, ns, slots, p0s, dev), out, 7)
    torch.cuda.synchronize()
    got = out.cpu()
    assert torch.isfinite(got.float()).all()
    err = maxabs(got, want)
    say(f"  max-abs {err:.3e}")
    assert err <= TOL


def test_prefill_graph_mode_plan(a8, ref, dev):
    """The graph-mode plan buffer (padding blocks point at the scratch row with n = 0) gives the same rows as
    an exact PrefillPlan, and leaves rows past the packed tokens untouched."""
    say("case: prefill graph-mode plan with padding")
    g = torch.Generator().manual_seed(32)
    NT, NR, rows, S = 512, 8, 6, 400
    SCR = rows - 1
    slots, ns, starts = [0, 3, 1], [130, 7, 64], [200, 0, 17]
    nt = 256
    q = randn_bf16(g, NT, NQ, HD)
    kc, vc = randn_bf16(g, rows, NKV, S, HD), randn_bf16(g, rows, NKV, S, HD)
    meta = a8.PrefillMeta(NT, NR, SCR, dev)
    meta.load(nt, slots, ns, starts)
    sentinel = torch.full((NT, NQ, HD), 7.0, dtype=BF, device=dev)
    out = sentinel.clone()
    a8.prefill_attention(q.to(dev)[:nt], kc.to(dev), vc.to(dev), meta.plan(nt), out[:nt], 7)
    torch.cuda.synchronize()
    r0s = [0, 130, 137]
    want = torch.zeros(NT, NQ, HD, dtype=BF)
    ref.prefill_attention(q, kc, vc, *ref.prefill_plan(r0s, ns, slots, starts), want, 7)
    R = sum(ns)
    assert maxabs(out[:R], want[:R]) <= TOL
    assert torch.equal(out[R:].cpu(), sentinel[R:].cpu())


def test_prefill_graph_replay_admissions(a8, ref, dev):
    """The engine's prefill graph per token bucket (fast_engine.py:797-812, 820-853, 1109-1116): the stack's
    store + prefill captured once over a PrefillMeta buffer, then replayed for admissions with other slots,
    lengths and prefixes (each written by one host-to-device copy, and each admission's prefix K/V put into
    its slots by prefix_copy first). Every replay equals the eager forward on the same inputs bit for bit, and
    the eager forward matches the oracle."""
    say("case: prefill graph captured once, replayed for three admissions")
    g = torch.Generator().manual_seed(35)
    NT, NR, rows, S, layers = 512, 8, 9, 640, 2
    SCR = rows - 1
    W = (NQ + 2 * NKV) * HD
    st = a8.AttnStack(layers, NQ, NKV, HD, 10000.0, max_rows=NT, cache_rows=rows, cache_len=S, max_pos=S, dev=dev)
    meta = a8.PrefillMeta(NT, NR, SCR, dev)
    nt = 512
    qkv = [torch.zeros(NT, W, dtype=BF, device=dev) for _ in range(layers)]
    bias = [randn_bf16(g, W, std=0.02).to(dev) for _ in range(layers)]
    q = torch.empty(NT, NQ, HD, dtype=BF, device=dev)
    outs = [torch.zeros(NT, NQ, HD, dtype=BF, device=dev) for _ in range(layers)]
    v = meta.v

    def body():
        st.forward(qkv, bias, v.pos[:nt], v.slot[:nt], None, plan=meta.plan(nt), q=q, outs=outs)

    admissions = [([0, 3, 1], [130, 7, 64], [200, 0, 17]), ([5, 2], [300, 190], [100, 0]),
                  ([7, 6, 4, 0, 1], [1, 64, 65, 100, 250], [300, 300, 0, 20, 300])]
    meta.load(nt, *admissions[0])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()
    torch.cuda.synchronize()
    prefix_k = randn_bf16(g, layers, NKV, 300, HD).to(dev)
    prefix_v = randn_bf16(g, layers, NKV, 300, HD).to(dev)
    for slots, ns, starts in admissions:
        R = sum(ns)
        kc0 = randn_bf16(g, layers, rows, NKV, S, HD).to(dev)
        vc0 = randn_bf16(g, layers, rows, NKV, S, HD).to(dev)
        x = [randn_bf16(g, R, W).to(dev) for _ in range(layers)]
        res = []
        for mode in ("graph", "eager"):
            st.kc_all.copy_(kc0)
            st.vc_all.copy_(vc0)
            a8.prefix_copy(prefix_k, prefix_v, st.kc_all, st.vc_all, [s_ for s_, a in zip(slots, starts) if a == 300])
            meta.load(nt, slots, ns, starts)
            for i in range(layers):
                qkv[i].zero_()
                qkv[i][:R].copy_(x[i])
                outs[i].zero_()
            if mode == "graph":
                graph.replay()
            else:
                body()
            torch.cuda.synchronize()
            res.append(([o[:R].cpu() for o in outs], st.kc_all.cpu(), st.vc_all.cpu()))
        (og, kg, vg), (oe, ke, ve) = res
        assert all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(og, oe))
        assert torch.equal(kg.view(torch.int16), ke.view(torch.int16))
        assert torch.equal(vg.view(torch.int16), ve.view(torch.int16))
        # the oracle on the last layer: the initial cache, the prefix put into its slots, the store, the prefill
        r0s = [int(r) for r in np.cumsum([0] + ns[:-1])]
        qo = torch.zeros(R, NQ, HD, dtype=BF)
        pos = torch.cat([torch.arange(a, a + n) for a, n in zip(starts, ns)]).int()
        slot = torch.cat([torch.full((n,), s_) for s_, n in zip(slots, ns)]).int()
        kl, vl = kc0[layers - 1].cpu(), vc0[layers - 1].cpu()
        for s_, a in zip(slots, starts):
            if a == 300:
                kl[s_, :, :300] = prefix_k[layers - 1].cpu()
                vl[s_, :, :300] = prefix_v[layers - 1].cpu()
        cos, sin = ref.rope_tables(10000.0, HD, S)
        ref.bias_rope_store(x[layers - 1].cpu(), bias[layers - 1].cpu(), cos, sin, pos, slot, qo, kl, vl, NQ, NKV, HD)
        # (the padding rows store into the scratch row SCR, as in the reference; the other rows must match)
        assert torch.equal(kl[:SCR].view(torch.int16), ke[layers - 1, :SCR].view(torch.int16))
        assert torch.equal(vl[:SCR].view(torch.int16), ve[layers - 1, :SCR].view(torch.int16))
        want = torch.zeros(R, NQ, HD, dtype=BF)
        ref.prefill_attention(qo, kl, vl, *ref.prefill_plan(r0s, ns, slots, starts), want, NQ // NKV)
        assert maxabs(oe[layers - 1], want) <= TOL


def test_prefill_rows_match_decode(a8, dev):
    """HIP prefill row j == HIP decode with lens = p0 + j + 1 on the same cache row (two independent kernels)."""
    say("case: prefill vs decode cross-check")
    g = torch.Generator().manual_seed(33)
    rows, S = 3, 512
    kc, vc = randn_bf16(g, rows, NKV, S, HD).to(dev), randn_bf16(g, rows, NKV, S, HD).to(dev)
    ns, p0s, slots = [150, 64, 1], [300, 0, 511], [2, 0, 1]
    r0s = [0, 150, 214]
    R = sum(ns)
    q = randn_bf16(g, R, NQ, HD).to(dev)
    out = torch.zeros(R, NQ, HD, dtype=BF, device=dev)
    a8.prefill_attention(q, kc, vc, a8.PrefillPlan(r0s, ns, slots, p0s, dev), out, 7)
    lens = torch.tensor([p0 + j + 1 for n, p0 in zip(ns, p0s) for j in range(n)], dtype=torch.int32, device=dev)
    rowmap = torch.tensor([s for n, s in zip(ns, slots) for _ in range(n)], dtype=torch.int32, device=dev)
    att = a8.DecodeAttention(16 * R, NQ, NKV, HD, 16, dev)
    dec = torch.empty_like(out)
    att(q, kc, vc, lens, dec, nsplit=2, rowmap=rowmap)
    torch.cuda.synchronize()
    assert maxabs(out, dec) <= TOL


@pytest.mark.parametrize("nq,nkv", [(14, 2), (10, 2), (12, 2), (16, 2), (16, 1), (8, 2), (4, 4)])
def test_prefill_groups(a8, ref, dev, nq, nkv):
    """Every head grouping through the workgroup shapes it takes (q heads per kv head split into shares of <= 4
    waves: 7 -> 4 + 3, 5 -> 4 + 1, 6 -> 4 + 2, 16 -> 4 x 4; 1 and 2 in one workgroup) against the oracle: 200
    short requests (one-tile blocks, last query groups empty), 24 long ones, and padding blocks (n = 0)
    between them; rows past the packed tokens stay untouched."""
    group = nq // nkv
    say(f"case: prefill nq={nq} nkv={nkv} (group {group})")
    g = torch.Generator().manual_seed(40 + group * 3 + nkv)
    S = 704
    ns = torch.randint(1, 65, (200,), generator=g).tolist() + torch.randint(100, 301, (24,), generator=g).tolist()
    p0s = torch.randint(0, 101, (200,), generator=g).tolist() + torch.randint(0, 301, (24,), generator=g).tolist()
    nreq = len(ns)
    slots = torch.randperm(nreq, generator=g).tolist()
    r0s = [int(x) for x in np.cumsum([0] + ns[:-1])]
    R = sum(ns)
    kc, vc = randn_bf16(g, nreq + 1, nkv, S, HD), randn_bf16(g, nreq + 1, nkv, S, HD)
    q = randn_bf16(g, R + 64, nq, HD)
    want = torch.zeros(R, nq, HD, dtype=BF)
    ref.prefill_attention(q[:R], kc, vc, *ref.prefill_plan(r0s, ns, slots, p0s), want, group)
    # the plan's blocks with a padding block (n = 0, rows R..R+63 of the scratch slot) after every 16th
    plan = a8.PrefillPlan(r0s, ns, slots, p0s, dev)
    cols = [t.cpu().tolist() for t in (plan.q0, plan.n, plan.slot, plan.pos0)]
    blocks = []
    for i, b in enumerate(zip(*cols)):
        blocks.append(b)
        if i % 16 == 15:
            blocks.append((R, 0, nreq, 0))
    t = torch.tensor(blocks, dtype=torch.int32).T.contiguous().to(dev)

    class Plan:
        BM, nblk = 64, len(blocks)
        q0, n, slot, pos0 = t[0], t[1], t[2], t[3]

    out = torch.full((R + 64, nq, HD), 7.0, dtype=BF, device=dev)
    a8.prefill_attention(q.to(dev), kc.to(dev), vc.to(dev), Plan, out, group)
    torch.cuda.synchronize()
    got = out.cpu()
    err = maxabs(got[:R], want)
    say(f"  R={R} blocks={len(blocks)} max-abs {err:.3e}")
    assert torch.isfinite(got[:R].float()).all()
    assert err <= TOL
    assert (got[R:].float() == 7.0).all()


def _bits(a, b):
    return torch.equal(a.cpu().view(torch.int16), b.cpu().view(torch.int16))


def _store_prefill_both(a8, dev, qkv, bias, cos, sin, pos, slot, kc, vc, plan, nq, nkv, R):
    """bias_rope_store + prefill_attention against bias_rope_store(qo=None) + prefill_attention_qkv on copies of
    the same caches: (out, kc, vc, q) of the first, (out, kc, vc) of the second."""
    res = []
    for fused in (False, True):
        kd, vd = kc.clone(), vc.clone()
        out = torch.full((R, nq, HD), 7.0, dtype=BF, device=dev)
        if fused:
            a8.bias_rope_store(qkv, bias, cos, sin, pos, slot, None, kd, vd, nq, nkv, HD)
            a8.prefill_attention_qkv(qkv, bias, cos, sin, kd, vd, plan, out, nq // nkv)
            res.append((out, kd, vd))
        else:
            q = torch.zeros(R, nq, HD, dtype=BF, device=dev)
            a8.bias_rope_store(qkv, bias, cos, sin, pos, slot, q, kd, vd, nq, nkv, HD)
            a8.prefill_attention(q, kd, vd, plan, out, nq // nkv)
            res.append((out, kd, vd, q))
    torch.cuda.synchronize()
    return res


def test_prefill_qkv_c4_matches_unfused(a8, ref, dev):
    """Config 4 at full size: the store (k / v only) + the prefill forming q from the qkv rows leave the same
    out and cache bits as the store (q, k, v) + the prefill over the stored q, and the out is within the bar of
    the oracle's."""
    say("case: fused-q prefill C4 full size vs store + prefill")
    g = torch.Generator().manual_seed(36)
    ns, S, pk, pv = _c4(g)
    p0, nreq = 300, len(ns)
    W = (NQ + 2 * NKV) * HD
    R = sum(ns)
    qkv, bias = randn_bf16(g, R, W), randn_bf16(g, W, std=0.02)
    cos, sin = ref.rope_tables(10000.0, HD, 2048)
    pos = torch.cat([p0 + torch.arange(n) for n in ns]).int()
    slot = torch.cat([torch.full((n,), i) for i, n in enumerate(ns)]).int()
    r0s = [int(x) for x in np.cumsum([0] + ns[:-1])]
    kc = torch.zeros(nreq + 1, NKV, S, HD, dtype=BF)
    vc = torch.zeros_like(kc)
    for i in range(nreq):
        kc[i, :, :p0], vc[i, :, :p0] = pk[i % 4], pv[i % 4]
    plan = a8.PrefillPlan(r0s, ns, list(range(nreq)), [p0] * nreq, dev)
    (o1, k1, v1, q1), (o2, k2, v2) = _store_prefill_both(
        a8, dev, qkv.to(dev), bias.to(dev), cos.to(dev), sin.to(dev), pos.to(dev), slot.to(dev), kc.to(dev),
        vc.to(dev), plan, NQ, NKV, R)
    assert _bits(o1, o2) and _bits(k1, k2) and _bits(v1, v2)
    q_c = torch.empty(R, NQ, HD, dtype=BF)
    ref.bias_rope_store(qkv, bias, cos, sin, pos, slot, q_c, kc, vc, NQ, NKV, HD)
    want = torch.zeros(R, NQ, HD, dtype=BF)
    ref.prefill_attention(q_c, kc, vc, *ref.prefill_plan(r0s, ns, list(range(nreq)), [p0] * nreq), want, 7)
    err = maxabs(o2, want)
    say(f"  R={R} blocks={plan.nblk} bits equal, max-abs vs oracle {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("nq,nkv,with_bias", [(14, 2, True), (14, 2, False), (16, 1, True), (8, 2, True),
                                              (4, 4, True), (10, 2, False), (12, 2, True)])
def test_prefill_qkv_groups(a8, ref, dev, nq, nkv, with_bias):
    """The fused-q prefill over every workgroup shape, with padding blocks (n = 0) in the plan, qkv rows wider
    than the projection (row stride W + 64), and RoPE tables of 400 positions that end inside some requests
    (the store writes nothing for those rows; the unfused q rows stay 0, the fused prefill attends with q = 0):
    the same out and cache bits as the unfused pair, rows past the packed tokens untouched, and the out within
    the bar of the oracle's."""
    group = nq // nkv
    say(f"case: fused-q prefill nq={nq} nkv={nkv} bias={with_bias}")
    g = torch.Generator().manual_seed(60 + 3 * group + nkv + (7 if with_bias else 0))
    S, n_tab = 704, 400
    ns = torch.randint(1, 65, (40,), generator=g).tolist() + torch.randint(100, 301, (8,), generator=g).tolist()
    p0s = torch.randint(0, 101, (40,), generator=g).tolist() + torch.randint(0, 301, (8,), generator=g).tolist()
    ns, p0s = ns + [120], p0s + [350]  # a request running past the tables
    nreq = len(ns)
    slots = torch.randperm(nreq, generator=g).tolist()
    r0s = [int(x) for x in np.cumsum([0] + ns[:-1])]
    R = sum(ns)
    W = (nq + 2 * nkv) * HD
    wide = randn_bf16(g, R, W + 64)
    bias = randn_bf16(g, W, std=0.02) if with_bias else None
    cos, sin = ref.rope_tables(10000.0, HD, n_tab)
    pos = torch.cat([a + torch.arange(n) for a, n in zip(p0s, ns)]).int()
    slot = torch.cat([torch.full((n,), s_) for s_, n in zip(slots, ns)]).int()
    kc, vc = randn_bf16(g, nreq + 1, nkv, S, HD), randn_bf16(g, nreq + 1, nkv, S, HD)
    plan = a8.PrefillPlan(r0s, ns, slots, p0s, dev)
    cols = [t.cpu().tolist() for t in (plan.q0, plan.n, plan.slot, plan.pos0)]
    blocks = []
    for i, b in enumerate(zip(*cols)):
        blocks.append(b)
        if i % 8 == 7:
            blocks.append((R, 0, nreq, 0))
    t = torch.tensor(blocks, dtype=torch.int32).T.contiguous().to(dev)

    class Plan:
        BM, nblk = 64, len(blocks)
        q0, n, slot, pos0 = t[0], t[1], t[2], t[3]

    assert int(pos.max()) >= n_tab  # some rows past the tables
    qkv_d = wide.to(dev)[:, :W]
    (o1, k1, v1, q1), (o2, k2, v2) = _store_prefill_both(
        a8, dev, qkv_d, bias.to(dev) if bias is not None else None, cos.to(dev), sin.to(dev), pos.to(dev),
        slot.to(dev), kc.to(dev), vc.to(dev), Plan, nq, nkv, R)
    assert _bits(o1, o2) and _bits(k1, k2) and _bits(v1, v2)
    # the oracle's store on the rows inside the tables (it indexes the tables by position)
    keep = pos < n_tab
    q_in = torch.zeros(int(keep.sum()), nq, HD, dtype=BF)
    kl, vl = kc.clone(), vc.clone()
    ref.bias_rope_store(wide[keep][:, :W], bias, cos, sin, pos[keep], slot[keep], q_in, kl, vl, nq, nkv, HD)
    q_c = torch.zeros(R, nq, HD, dtype=BF)
    q_c[keep] = q_in
    assert _bits(q1, q_c) and _bits(k2, kl) and _bits(v2, vl)
    want = torch.zeros(R, nq, HD, dtype=BF)
    ref.prefill_attention(q_c, kl, vl, *ref.prefill_plan(r0s, ns, slots, p0s), want, group)
    err = maxabs(o2, want)
    say(f"  R={R} blocks={len(blocks)} bits equal, max-abs vs oracle {err:.3e}")
    assert torch.isfinite(o2.float()).all() and err <= TOL


def test_attn_stack_prefill_fused_graph(a8, dev):
    """AttnStack.forward with a plan and fuse=True (k / v stored, q formed inside the prefill), captured in a
    graph over a PrefillMeta buffer and replayed for two admissions: every replay equals the unfused eager
    forward (q written, then read) bit for bit in out and caches."""
    say("case: stack prefill fused-q, graph replays vs unfused eager")
    g = torch.Generator().manual_seed(37)
    NT, NR, rows, S, layers = 512, 8, 9, 640, 2
    W = (NQ + 2 * NKV) * HD
    st = a8.AttnStack(layers, NQ, NKV, HD, 10000.0, max_rows=NT, cache_rows=rows, cache_len=S, max_pos=S, dev=dev)
    meta = a8.PrefillMeta(NT, NR, rows - 1, dev)
    nt = 512
    qkv = [torch.zeros(NT, W, dtype=BF, device=dev) for _ in range(layers)]
    bias = [randn_bf16(g, W, std=0.02).to(dev) for _ in range(layers)]
    q = torch.zeros(NT, NQ, HD, dtype=BF, device=dev)
    outs = [torch.zeros(NT, NQ, HD, dtype=BF, device=dev) for _ in range(layers)]
    v = meta.v

    def body(fuse):
        st.forward(qkv, bias, v.pos[:nt], v.slot[:nt], None, plan=meta.plan(nt), q=q, outs=outs, fuse=fuse)

    admissions = [([0, 3, 1], [130, 7, 64], [200, 0, 17]), ([7, 6, 4, 0, 1], [1, 64, 65, 100, 250],
                                                             [300, 300, 0, 20, 300])]
    meta.load(nt, *admissions[0])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body(True)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body(True)
    torch.cuda.synchronize()
    for slots, ns, starts in admissions:
        R = sum(ns)
        kc0 = randn_bf16(g, layers, rows, NKV, S, HD).to(dev)
        vc0 = randn_bf16(g, layers, rows, NKV, S, HD).to(dev)
        x = [randn_bf16(g, R, W).to(dev) for _ in range(layers)]
        res = []
        for mode in ("graph", "unfused"):
            st.kc_all.copy_(kc0)
            st.vc_all.copy_(vc0)
            meta.load(nt, slots, ns, starts)
            for i in range(layers):
                qkv[i].zero_()
                qkv[i][:R].copy_(x[i])
                outs[i].zero_()
            if mode == "graph":
                graph.replay()
            else:
                body(False)
            torch.cuda.synchronize()
            res.append(([o[:R].cpu() for o in outs], st.kc_all.cpu(), st.vc_all.cpu()))
        (og, kg, vg), (oe, ke, ve) = res
        assert all(_bits(a, b) for a, b in zip(og, oe))
        assert _bits(kg, ke) and _bits(vg, ve)
        say(f"  admission {slots}: graph replay == unfused eager")
