"""Pins the CPU oracle (oracle/attn_ref.py) without retyping it: against the golden vectors written by
tests/golden/make_golden.py (numpy, float64 / float32, independent of the oracle), against closed forms
and against invariants that a dropped term, a wrong sign or index, or a transposed operand would break."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import bf16_from_bits, bits_of, golden, randn_bf16

BF = torch.bfloat16


def bf16_ulp(x):
    """Spacing of bf16 numbers at |x| (x float64 array)."""
    ax = np.maximum(np.abs(x), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(ax)) - 7)


# ---------------------------------------------------------------- a1: RoPE tables
def test_rope_tables_closed_form(ref):
    z = golden("rope.npz")
    base, hd, n = float(z["base"]), int(z["hd"]), int(z["n"])
    cos, sin = ref.rope_tables(base, hd, n)
    assert cos.shape == (n, hd) and sin.shape == (n, hd) and cos.dtype == BF
    pos = z["pos"]
    for tab, exact in ((cos, z["cos64"]), (sin, z["sin64"])):
        t = tab.float().numpy()[pos]
        # rotate_half tables repeat the 32 frequencies in both halves
        np.testing.assert_array_equal(t[:, :hd // 2], t[:, hd // 2:])
        # bf16 rounding (half an ulp) plus the fp32 phase error (<= |phase| * 2^-22 after two roundings)
        phase = np.outer(pos.astype(np.float64), base ** (-2.0 * np.arange(hd // 2) / hd))
        bound = 0.5 * bf16_ulp(exact.astype(np.float64)) + phase * 2.0 ** -22 + 1e-7
        err = np.abs(t[:, :hd // 2] - exact.astype(np.float64))
        assert (err <= bound).all(), float((err - bound).max())


def test_rope_tables_special_values(ref):
    cos, sin = ref.rope_tables(10000.0, 64, 8)
    assert torch.equal(cos[0], torch.ones(64, dtype=BF)) and torch.equal(sin[0], torch.zeros(64, dtype=BF))
    # frequency 0 is 1 rad / position: cos(1), sin(1) rounded to bf16
    assert cos[1, 0].item() == torch.tensor(math.cos(1.0)).to(BF).item()
    assert sin[1, 0].item() == torch.tensor(math.sin(1.0)).to(BF).item()


# ---------------------------------------------------------------- a2: permutation
def _interleaved_rope(x, pos, base, hd):
    """Textbook interleaved RoPE on pairs (2i, 2i+1), float64."""
    i = np.arange(hd // 2)
    th = pos * base ** (-2.0 * i / hd)
    c, s = np.cos(th), np.sin(th)
    x0, x1 = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = x0 * c - x1 * s
    out[..., 1::2] = x0 * s + x1 * c
    return out


def _rotate_half(x, pos, base, hd):
    """o[d] = x[d] cos + sign(d) x[(d+hd/2) % hd] sin with sign -1 below hd/2 (the store's formula), float64."""
    i = np.arange(hd) % (hd // 2)
    th = pos * base ** (-2.0 * i / hd)
    d = np.arange(hd)
    sign = np.where(d < hd // 2, -1.0, 1.0)
    return x * np.cos(th) + sign * x[..., (d + hd // 2) % hd] * np.sin(th)


def test_permute_qk_preserves_scores(ref):
    nq, nkv, hd, K = 14, 2, 64, 5
    g = torch.Generator().manual_seed(1)
    W = torch.randn((nq + 2 * nkv) * hd, K, generator=g, dtype=torch.float64)
    b = torch.randn((nq + 2 * nkv) * hd, generator=g, dtype=torch.float64)
    Wp, bp = ref.permute_qk(W, nq, nkv, hd), ref.permute_qk(b, nq, nkv, hd)
    x = torch.randn(K, generator=g, dtype=torch.float64)
    y0 = (W @ x + b).numpy()
    y1 = (Wp @ x + bp).numpy()
    # v rows untouched, q/k rows a per-head permutation
    np.testing.assert_array_equal(y1[(nq + nkv) * hd:], y0[(nq + nkv) * hd:])
    for pq, pk in ((7, 300), (1234, 5), (0, 2047)):
        for h in range(nq):
            qi = y0[h * hd:(h + 1) * hd]
            qp = y1[h * hd:(h + 1) * hd]
            kh = h // (nq // nkv)
            ki = y0[(nq + kh) * hd:(nq + kh + 1) * hd]
            kp = y1[(nq + kh) * hd:(nq + kh + 1) * hd]
            want = _interleaved_rope(qi, pq, 10000.0, hd) @ _interleaved_rope(ki, pk, 10000.0, hd)
            got = _rotate_half(qp, pq, 10000.0, hd) @ _rotate_half(kp, pk, 10000.0, hd)
            assert abs(want - got) <= 1e-9 * (1 + abs(want))


# ---------------------------------------------------------------- a3: store
def _store_from_golden(ref, z):
    nq, nkv, hd = int(z["nq"]), int(z["nkv"]), int(z["hd"])
    sent = int(z["sentinel"])
    rows, S = int(z["rows"]), int(z["S"])
    kc = bf16_from_bits(np.full((rows, nkv, S, hd), sent, np.uint16)).clone()
    vc = kc.clone()
    qo = bf16_from_bits(np.full(z["qo"].shape, sent, np.uint16)).clone()
    ref.bias_rope_store(bf16_from_bits(z["qkv"]), bf16_from_bits(z["bias"]), bf16_from_bits(z["cos"]),
                        bf16_from_bits(z["sin"]), torch.from_numpy(z["pos"]), torch.from_numpy(z["slot"]), qo, kc,
                        vc, nq, nkv, hd, ring=int(z["ring"]))
    return qo, kc, vc


def test_store_golden_bit_exact(ref):
    z = golden("store.npz")
    qo, kc, vc = _store_from_golden(ref, z)
    np.testing.assert_array_equal(bits_of(qo), z["qo"])
    np.testing.assert_array_equal(bits_of(kc), z["kc"])
    np.testing.assert_array_equal(bits_of(vc), z["vc"])


def test_store_touches_only_slot_positions(ref):
    """Brute force: with a sentinel cache, exactly the [slot, :, pos % ring] rows change."""
    z = golden("store.npz")
    _, kc, vc = _store_from_golden(ref, z)
    sent = int(z["sentinel"])
    ring = int(z["ring"])
    want = {(int(s), int(p) % ring) for s, p in zip(z["slot"], z["pos"])}
    for cache in (kc, vc):
        changed = (bits_of(cache) != sent).any(-1)            # [rows, nkv, S]
        got = {(int(r), int(c)) for r, h, c in zip(*np.nonzero(changed))}
        assert got == want
        assert changed.sum() == len(want) * cache.shape[1]


def test_store_rotation_closed_form(ref):
    """q/k outputs equal the float64 rotation of (qkv + bias) to within bf16 rounding."""
    nq, nkv, hd = 14, 2, 64
    g = torch.Generator().manual_seed(3)
    R, W = 9, (nq + 2 * nkv) * hd
    qkv, bias = randn_bf16(g, R, W), randn_bf16(g, W, std=0.02)
    cos, sin = ref.rope_tables(10000.0, hd, 600)
    pos = torch.randint(0, 600, (R,), generator=g, dtype=torch.int32)
    slot = torch.arange(R, dtype=torch.int32)
    qo = torch.empty(R, nq, hd, dtype=BF)
    kc = torch.zeros(R, nkv, 600, hd, dtype=BF)
    vc = torch.zeros_like(kc)
    ref.bias_rope_store(qkv, bias, cos, sin, pos, slot, qo, kc, vc, nq, nkv, hd)
    x = (qkv.double() + bias.double()).view(R, nq + 2 * nkv, hd).numpy()
    c = cos.double().numpy()[pos.numpy()][:, None]
    s = sin.double().numpy()[pos.numpy()][:, None]
    d = np.arange(hd)
    sign = np.where(d < 32, -1.0, 1.0)
    rot = x[:, :nq + nkv] * c + sign * x[:, :nq + nkv][..., (d + 32) % hd] * s
    got_q = qo.double().numpy()
    got_k = np.stack([kc[r, :, pos[r]].double().numpy() for r in range(R)])
    got_v = np.stack([vc[r, :, pos[r]].double().numpy() for r in range(R)])
    for got, want in ((got_q, rot[:, :nq]), (got_k, rot[:, nq:]), (got_v, x[:, nq + nkv:])):
        assert (np.abs(got - want) <= bf16_ulp(want) * 0.5 + 1e-6 * np.abs(want) + 1e-30).all()


# ---------------------------------------------------------------- a5-a8: decode
def _golden_decode_inputs():
    z = golden("decode.npz")
    return (z, bf16_from_bits(z["q"]), bf16_from_bits(z["kc"]), bf16_from_bits(z["vc"]),
            torch.from_numpy(z["lens"]), torch.from_numpy(z["rowmap"]))


@pytest.mark.parametrize("nsplit", [1, 2, 3, 16])
def test_decode_golden(ref, nsplit):
    z, q, kc, vc, lens, rowmap = _golden_decode_inputs()
    out = ref.decode_attention(q, kc, vc, lens, nsplit=nsplit, rowmap=rowmap)
    err = np.abs(out.float().numpy() - z["out"]).max()
    assert err <= 1e-2, err


def test_decode_textbook_random(ref):
    """Random lengths incl. exact tile multiples, against a float64 full-softmax restatement."""
    g = torch.Generator().manual_seed(5)
    nq, nkv, hd, S, b = 14, 2, 64, 300, 7
    q = randn_bf16(g, b, nq, hd)
    kc, vc = randn_bf16(g, b, nkv, S, hd), randn_bf16(g, b, nkv, S, hd)
    lens = torch.tensor([1, 2, 63, 64, 65, 128, 300], dtype=torch.int32)
    out = ref.decode_attention(q, kc, vc, lens, nsplit=4).double()
    for i in range(b):
        L = int(lens[i])
        for h in range(nq):
            K, V = kc[i, h // 7, :L].double(), vc[i, h // 7, :L].double()
            p = torch.softmax(K @ q[i, h].double() / 8.0, 0)
            assert (out[i, h] - p @ V).abs().max() <= 1e-2


def test_decode_special_cases(ref):
    g = torch.Generator().manual_seed(6)
    nq, nkv, hd, S = 14, 2, 64, 130
    q = randn_bf16(g, 3, nq, hd)
    kc, vc = randn_bf16(g, 3, nkv, S, hd), randn_bf16(g, 3, nkv, S, hd)
    # L = 1: the single value row, exactly, for any split count
    for ns in (1, 5):
        out = ref.decode_attention(q, kc, vc, torch.tensor([1, 1, 1], dtype=torch.int32), nsplit=ns)
        for i in range(3):
            assert torch.equal(out[i, :7], vc[i, 0, 0].expand(7, hd))
            assert torch.equal(out[i, 7:], vc[i, 1, 0].expand(7, hd))
    # identical keys: uniform weights -> mean of the values
    kc2 = kc[:, :, :1].expand(3, nkv, S, hd).contiguous()
    out = ref.decode_attention(q, kc2, vc, torch.tensor([130, 77, 64], dtype=torch.int32), nsplit=3)
    for i, L in enumerate((130, 77, 64)):
        mean = vc[i, :, :L].double().mean(1)                         # [nkv, hd]
        want = mean.repeat_interleave(7, 0)
        assert (out[i].double() - want).abs().max() <= 4e-3
    # L = 0: 0/0 in the combine, as in the reference
    out = ref.decode_attention(q, kc, vc, torch.tensor([0, 5, 0], dtype=torch.int32), nsplit=2)
    assert torch.isnan(out[0].float()).all() and torch.isnan(out[2].float()).all()
    assert not torch.isnan(out[1].float()).any()


def test_decode_invariants(ref):
    g = torch.Generator().manual_seed(7)
    nq, nkv, hd, S, rows = 14, 2, 64, 200, 4
    q = randn_bf16(g, 5, nq, hd)
    kc, vc = randn_bf16(g, rows, nkv, S, hd), randn_bf16(g, rows, nkv, S, hd)
    lens = torch.tensor([200, 150, 3, 64, 129], dtype=torch.int32)
    rowmap = torch.tensor([3, 0, 2, 2, 1], dtype=torch.int32)
    outs = [ref.decode_attention(q, kc, vc, lens, nsplit=ns, rowmap=rowmap).float() for ns in (1, 2, 4, 16)]
    for o in outs[1:]:
        assert (o - outs[0]).abs().max() <= 1e-2
    # rowmap == gathering the cache rows
    gathered = ref.decode_attention(q, kc[rowmap.long()], vc[rowmap.long()], lens, nsplit=2)
    assert torch.equal(gathered, ref.decode_attention(q, kc, vc, lens, nsplit=2, rowmap=rowmap))
    # permuting key positions inside [0, L) leaves the softmax unchanged
    perm = torch.randperm(200, generator=g)
    kp, vp = kc.clone(), vc.clone()
    kp[:, :, :200], vp[:, :, :200] = kc[:, :, perm], vc[:, :, perm]
    full = torch.full((5,), 200, dtype=torch.int32)
    a = ref.decode_attention(q, kc, vc, full, nsplit=3, rowmap=rowmap).float()
    b = ref.decode_attention(q, kp, vp, full, nsplit=3, rowmap=rowmap).float()
    assert (a - b).abs().max() <= 1e-2


def test_ref_nsplit_table(ref):
    want = {1: 16, 2: 16, 4: 16, 8: 11, 16: 6, 32: 3, 64: 2, 128: 1, 192: 1}
    assert {b: ref.ref_nsplit(b, 2) for b in want} == want


# ---------------------------------------------------------------- a9-a11: prefill
def test_prefill_golden(ref):
    z = golden("prefill.npz")
    q, kc, vc = bf16_from_bits(z["q"]), bf16_from_bits(z["kc"]), bf16_from_bits(z["vc"])
    reqs = z["reqs"]
    ns = [int(n) for _, _, n in reqs]
    r0s = list(np.cumsum([0] + ns[:-1]))
    plan = ref.prefill_plan(r0s, ns, [int(s) for s, _, _ in reqs], [int(p) for _, p, _ in reqs])
    out = torch.zeros_like(q)
    ref.prefill_attention(q, kc, vc, *plan, out, 7)
    err = np.abs(out.float().numpy() - z["out"].astype(np.float64)).max()
    assert err <= 1e-2, err


def test_prefill_row_equals_decode(ref):
    """Row j of a request attends exactly what decode with lens = p0 + j + 1 attends."""
    g = torch.Generator().manual_seed(8)
    nq, nkv, hd, S = 14, 2, 64, 260
    kc, vc = randn_bf16(g, 2, nkv, S, hd), randn_bf16(g, 2, nkv, S, hd)
    ns, p0s, slots = [100, 37], [150, 0], [1, 0]
    R = sum(ns)
    q = randn_bf16(g, R, nq, hd)
    out = torch.zeros(R, nq, hd, dtype=BF)
    ref.prefill_attention(q, kc, vc, *ref.prefill_plan([0, 100], ns, slots, p0s), out, 7)
    lens = torch.tensor([p0s[0] + j + 1 for j in range(100)] + [j + 1 for j in range(37)], dtype=torch.int32)
    rowmap = torch.tensor([1] * 100 + [0] * 37, dtype=torch.int32)
    dec = ref.decode_attention(q, kc, vc, lens, nsplit=1, rowmap=rowmap)
    assert (out.float() - dec.float()).abs().max() <= 1e-2


def test_prefill_plan_brute_force(ref):
    rng = np.random.default_rng(9)
    ns = [int(x) for x in rng.integers(1, 300, 12)]
    r0s = list(np.cumsum([0] + ns[:-1]))
    slots = [int(x) for x in rng.integers(0, 50, 12)]
    p0s = [int(x) for x in rng.integers(0, 400, 12)]
    q0, cnt, sl, ps = ref.prefill_plan(r0s, ns, slots, p0s)
    assert len(q0) == sum(-(-n // 64) for n in ns)
    seen = {}
    for a, n, s, p in zip(q0, cnt, sl, ps):
        assert 1 <= n <= 64
        for j in range(n):
            assert a + j not in seen
            seen[a + j] = (s, p + j)
    # every packed row once, at its request's slot and position
    want = {}
    for r0, n, s, p0 in zip(r0s, ns, slots, p0s):
        for j in range(n):
            want[r0 + j] = (s, p0 + j)
    assert seen == want


def test_pf_meta_host_brute_force(ref):
    NT, NR, SCR = 512, 8, 99
    slots, ns, starts = [3, 7, 1], [70, 5, 130], [300, 0, 12]
    m = ref.pf_meta_host(256, slots, ns, starts, NT, NR, SCR)
    o = ref.pf_layout(NT, NR)
    f = {k: m[o[i]:o[i + 1]] for i, k in enumerate(("pos", "slot", "q0", "n", "bslot", "pos0", "last", "st", "cpos"))}
    r = 0
    for s, n, a in zip(slots, ns, starts):
        assert list(f["pos"][r:r + n]) == list(range(a, a + n)) and set(f["slot"][r:r + n]) == {s}
        r += n
    assert set(f["slot"][r:]) == {SCR} and not f["pos"][r:].any()
    blocks = [(int(a), int(b), int(c), int(d)) for a, b, c, d in zip(f["q0"], f["n"], f["bslot"], f["pos0"]) if b > 0]
    assert blocks == list(zip(*ref.prefill_plan([0, 70, 75], ns, slots, starts)))
    assert (f["n"][len(blocks):] == 0).all() and (f["bslot"][len(blocks):] == SCR).all()
    assert list(f["last"][:3]) == [69, 74, 204] and list(f["st"][:3]) == slots and list(f["cpos"][:3]) == [370, 5, 142]
    assert set(f["st"][3:]) == {SCR}
    with pytest.raises(AssertionError):
        ref.pf_meta_host(64, slots, ns, starts, NT, NR, SCR)     # 205 tokens do not fit a 64-token bucket


def test_algorithmic_counts(ref):
    """The byte / FLOP counts bench.py divides by: C3 per layer and a hand-checkable prefill case."""
    assert ref.decode_bytes([2048] * 192, 14, 2, 64) == 201_326_592 + 688_128 + 986_880
    assert ref.prefill_flops([2], [3], 14, 64) == 4 * 14 * 64 * (4 + 5)
