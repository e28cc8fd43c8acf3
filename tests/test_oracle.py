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


@pytest.mark.parametrize("hd", [64, 128])
def test_store_rotation_closed_form(ref, hd):
    """q/k outputs equal the float64 rotation of (qkv + bias) to within bf16 rounding (the engine's head_dim
    and 128, which the reference's generic-HD kernel also serves)."""
    nq, nkv = 14, 2
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
    sign = np.where(d < hd // 2, -1.0, 1.0)
    rot = x[:, :nq + nkv] * c + sign * x[:, :nq + nkv][..., (d + hd // 2) % hd] * s
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


@pytest.mark.parametrize("hd", [64, 128])
def test_decode_textbook_random(ref, hd):
    """Random lengths incl. exact tile multiples, against a float64 full-softmax restatement."""
    g = torch.Generator().manual_seed(5)
    nq, nkv, S, b = 14, 2, 300, 7
    q = randn_bf16(g, b, nq, hd)
    kc, vc = randn_bf16(g, b, nkv, S, hd), randn_bf16(g, b, nkv, S, hd)
    lens = torch.tensor([1, 2, 63, 64, 65, 128, 300], dtype=torch.int32)
    out = ref.decode_attention(q, kc, vc, lens, nsplit=4).double()
    for i in range(b):
        L = int(lens[i])
        for h in range(nq):
            K, V = kc[i, h // 7, :L].double(), vc[i, h // 7, :L].double()
            p = torch.softmax(K @ q[i, h].double() * hd ** -0.5, 0)
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


@pytest.mark.parametrize("hd", [64, 128])
def test_prefill_row_equals_decode(ref, hd):
    """Row j of a request attends exactly what decode with lens = p0 + j + 1 attends."""
    g = torch.Generator().manual_seed(8)
    nq, nkv, S = 14, 2, 260
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


# ---- the slow-AR layer steps (oracle/layer_ref.py) ----

@pytest.fixture(scope="module")
def lref():
    from oracle import layer_ref
    return layer_ref


def _ulps(a, b):
    """bf16 distance in units in the last place (same-sign finite values)."""
    return (a.view(torch.int16).int() - b.view(torch.int16).int()).abs()


def test_layer_rmsnorm_against_library(lref):
    g = torch.Generator().manual_seed(61)
    for N in (896, 1024):
        x, r = randn_bf16(g, 64, N, std=3.0), randn_bf16(g, 64, N)
        w = (1 + 0.1 * torch.randn(N, generator=g)).to(torch.bfloat16)
        y, h = lref.rmsnorm(x, w, 1e-6, residual=r)
        h64 = x.double() + r.double()
        assert torch.equal(h, h64.to(torch.bfloat16))                       # one rounding of the exact sum
        xn = torch.nn.functional.rms_norm(h.double(), (N,), eps=1e-6).to(torch.bfloat16)
        want = (w.double() * xn.double()).to(torch.bfloat16)
        d = _ulps(y, want)
        assert d.max() <= 1 and (d == 0).float().mean() >= 0.995
        y0, h0 = lref.rmsnorm(x, w, 1e-6)                                     # no residual: h is x
        assert h0 is x and _ulps(y0, (w.double() * torch.nn.functional.rms_norm(
            x.double(), (N,), eps=1e-6).to(torch.bfloat16).double()).to(torch.bfloat16)).max() <= 1
    # a planted mistake (the weight applied before the bf16 rounding of xn) is caught
    x = randn_bf16(g, 64, 896, std=3.0)
    w = (1 + 0.1 * torch.randn(896, generator=g)).to(torch.bfloat16)
    wrong = (w.double() * torch.nn.functional.rms_norm(x.double(), (896,), eps=1e-6)).to(torch.bfloat16)
    assert (_ulps(lref.rmsnorm(x, w, 1e-6)[0], wrong) > 0).float().mean() > 0.05


def test_layer_silu_mul_against_library(lref):
    g = torch.Generator().manual_seed(62)
    gu = randn_bf16(g, 32, 2 * 1024, std=4.0)
    y = lref.silu_mul(gu)
    gs = torch.nn.functional.silu(gu[:, :1024].double()).to(torch.bfloat16)
    want = (gs.double() * gu[:, 1024:].double()).to(torch.bfloat16)
    d = _ulps(y, want)
    assert y.shape == (32, 1024) and d.max() <= 1 and (d == 0).float().mean() >= 0.995


def test_layer_linear_against_float64(lref):
    g = torch.Generator().manual_seed(63)
    x, w = randn_bf16(g, 16, 896), randn_bf16(g, 1152, 896)
    want = (x.double() @ w.double().t()).to(torch.bfloat16)
    d = _ulps(lref.linear(x, w), want)
    assert d.max() <= 1 and (d == 0).float().mean() >= 0.99


def test_layer_slow_stack_against_float64_unrolled(ref, lref):
    """One decode layer of the stack against a float64 evaluation written out step by step (textbook RMSNorm,
    GEMMs, RoPE on the rotate_half layout, softmax attention over the cache with the new key, SwiGLU, two
    residual adds, the final norm): agreement to bf16 rounding noise, and a dropped residual is caught."""
    g = torch.Generator().manual_seed(64)
    nq, nkv, hd, hidden, inter, S, b = 14, 2, 64, 896, 256, 64, 3
    W = (nq + 2 * nkv) * hd

    def lin(n, k):
        return (torch.randn(n, k, generator=g) / k ** 0.5).to(torch.bfloat16)

    L = dict(wqkv=lin(W, hidden), bqkv=randn_bf16(g, W, std=0.02), wo=lin(hidden, nq * hd), w13=lin(2 * inter, hidden),
             w2=lin(hidden, inter), ln1=(1 + 0.05 * torch.randn(hidden, generator=g)).to(torch.bfloat16),
             ln2=(1 + 0.05 * torch.randn(hidden, generator=g)).to(torch.bfloat16))
    norm = (1 + 0.05 * torch.randn(hidden, generator=g)).to(torch.bfloat16)
    x = randn_bf16(g, b, hidden)
    kc, vc = randn_bf16(g, b, nkv, S, hd), randn_bf16(g, b, nkv, S, hd)
    pos = torch.tensor([5, 40, 63], dtype=torch.int32)
    slot = torch.arange(b, dtype=torch.int32)
    lens = pos + 1
    cos, sin = ref.rope_tables(10000.0, hd, S)
    got = lref.slow_stack(x.clone(), pos, slot, lens, [L], norm, nq, nkv, hd, 1e-6, cos, sin, [kc.clone()],
                          [vc.clone()])

    def rms(v, w):
        return torch.nn.functional.rms_norm(v, (hidden,), eps=1e-6) * w.double()

    def rope(t, p):                      # rotate_half on [heads, hd] at position p
        c, s_ = cos[p].double(), sin[p].double()
        rot = torch.cat([-t[:, hd // 2:], t[:, :hd // 2]], -1)
        return t * c + rot * s_

    out = torch.empty(b, hidden, dtype=torch.float64)
    for r in range(b):
        p = int(pos[r])
        h0 = rms(x[r].double(), L["ln1"])
        qkv = L["wqkv"].double() @ h0 + L["bqkv"].double()
        q = rope(qkv[:nq * hd].view(nq, hd), p)
        k_new = rope(qkv[nq * hd:(nq + nkv) * hd].view(nkv, hd), p)
        v_new = qkv[(nq + nkv) * hd:].view(nkv, hd)
        K, V = kc[r].double().clone(), vc[r].double().clone()
        K[:, p], V[:, p] = k_new, v_new
        o = torch.empty(nq, hd, dtype=torch.float64)
        for hq in range(nq):
            kh = hq // (nq // nkv)
            s_ = K[kh, :p + 1] @ q[hq] / hd ** 0.5
            o[hq] = torch.softmax(s_, 0) @ V[kh, :p + 1]
        res1 = x[r].double() + L["wo"].double() @ o.reshape(-1)
        h1 = rms(res1, L["ln2"])
        gu = L["w13"].double() @ h1
        m = L["w2"].double() @ (torch.nn.functional.silu(gu[:inter]) * gu[inter:])
        out[r] = rms(res1 + m, norm)
    err = (got.double() - out).abs().max().item()
    assert err <= 0.02 * out.abs().max().item(), err   # measured 0.6 % (bf16 roundings of the stack)
    wrong = torch.stack([rms(out[r] * 0 + x[r].double(), norm) for r in range(b)])   # residual stream not updated
    assert (got.double() - wrong).abs().max().item() > 10 * err


def test_decode_fp32_query_against_float64(ref):
    """The oracle's decode with an fp32 query (the reference's PREC = "ieee" branch): against a float64
    textbook softmax attention over the same fp32 q and bf16 K / V, within the bf16 rounding of the weights
    that the reference applies before P.V; fp32 and bf16 outputs."""
    g = torch.Generator().manual_seed(31)
    b, nq, nkv, hd, S = 5, 6, 2, 64, 150
    q = torch.randn(b, nq, hd, generator=g)
    kc = torch.randn(b, nkv, S, hd, generator=g).to(torch.bfloat16)
    vc = torch.randn(b, nkv, S, hd, generator=g).to(torch.bfloat16)
    lens = torch.tensor([1, 64, 65, 100, 150], dtype=torch.int32)
    got = ref.decode_attention(q, kc, vc, lens, nsplit=3, out_dtype=torch.float32).double()
    got_bf = ref.decode_attention(q, kc, vc, lens, out_dtype=torch.bfloat16)
    assert got_bf.dtype == torch.bfloat16
    group = nq // nkv
    for r in range(b):
        L = int(lens[r])
        for h in range(nq):
            k = kc[r, h // group, :L].double()
            v = vc[r, h // group, :L].double()
            s = (k @ q[r, h].double()) * hd ** -0.5
            p = torch.softmax(s, 0)
            want = p @ v
            assert (got[r, h] - want).abs().max().item() <= 1e-2 * max(1.0, want.abs().max().item())
            assert (got_bf[r, h].double() - want).abs().max().item() <= 2e-2 * max(1.0, want.abs().max().item())


# ---- the vocoder's channels-last convolutions (oracle/conv_ref.py) ----

@pytest.fixture(scope="module")
def cref():
    from oracle import conv_ref
    return conv_ref


def test_conv_cl_against_conv1d(cref):
    """ph = 1: the causal dilated conv over a context-padded input equals torch's conv1d (cross-correlation)
    in float64 up to the one fp16 rounding; with bias, residual and the snake on the load."""
    g = torch.Generator().manual_seed(71)
    B, T, Cin, Cout, taps, dil = 3, 11, 32, 24, 7, 3
    Tin = T + (taps - 1) * dil
    x = (torch.randn(B, Tin, Cin, generator=g)).to(torch.float16)
    w = (torch.randn(1, taps, Cin, 32, generator=g) / 10).to(torch.float16)
    bias = torch.randn(Cout, generator=g).to(torch.float16)
    res = torch.randn(B, T, Cout, generator=g).to(torch.float16)
    a = torch.rand(Cin, generator=g) + 0.5
    ib = 1.0 / (a + 1e-9)
    got = cref.conv_cl(x, w, bias, T, taps, dil, 1, Cout, res=res, snake_ab=(a, ib))
    xs = cref.snake(x, a, ib)
    want = torch.nn.functional.conv1d(xs.double().transpose(1, 2), w[0, :, :, :Cout].double().permute(2, 1, 0),
                                      bias.double(), dilation=dil).transpose(1, 2)[:, :T] + res.double()
    assert (got.double() - want).abs().max().item() <= 2 ** -10 * want.abs().max().item()
    # a planted slip (taps read at stride 1 instead of dil) is caught
    slip = torch.nn.functional.conv1d(xs.double().transpose(1, 2), w[0, :, :, :Cout].double().permute(2, 1, 0),
                                      bias.double(), dilation=1).transpose(1, 2)[:, :T] + res.double()
    assert (got.double() - slip).abs().max().item() > 0.1


def test_conv_cl_phases_against_conv_transpose1d(cref):
    """ph = s: the phase split of a stride-s transposed conv (kernel 2s, right crop s: tap 0 = w[:, :, p+s]
    on the previous frame, tap 1 = w[:, :, p] on the current one, fast_engine.py:186-194) equals torch's
    conv_transpose1d cropped to the new frames."""
    g = torch.Generator().manual_seed(72)
    B, T, Cin, Cout, s = 2, 6, 16, 8, 4
    wt = (torch.randn(Cin, Cout, 2 * s, generator=g) / 4).to(torch.float16)
    W = torch.zeros(s, 2, Cin, Cout, dtype=torch.float16)
    for p in range(s):
        W[p, 0] = wt[:, :, p + s]
        W[p, 1] = wt[:, :, p]
    x = torch.randn(B, T + 1, Cin, generator=g).to(torch.float16)        # row 0: the previous frame
    got = cref.conv_cl(x, W, None, T, 2, 1, s, Cout)
    full = torch.nn.functional.conv_transpose1d(x.double().transpose(1, 2), wt.double(), stride=s)
    want = full[:, :, s:s + T * s].transpose(1, 2)
    assert (got.double() - want).abs().max().item() <= 2 ** -10 * want.abs().max().item()


def test_conv_cl_brute_force_tiny(cref):
    g = torch.Generator().manual_seed(73)
    B, T, Cin, Cout, taps, dil, ph = 2, 3, 8, 5, 2, 2, 3
    x = torch.randn(B, T + (taps - 1) * dil, Cin, generator=g).to(torch.float16)
    w = torch.randn(ph, taps, Cin, 8, generator=g).to(torch.float16)
    got = cref.conv_cl(x, w, None, T, taps, dil, ph, Cout)
    for b in range(B):
        for t in range(T):
            for p in range(ph):
                for n in range(Cout):
                    v = sum(float(x[b, t + j * dil, k]) * float(w[p, j, k, n]) for j in range(taps) for k in range(Cin))
                    assert abs(float(got[b, t * ph + p, n]) - v) <= 2 ** -10 * max(1.0, abs(v))


def test_snake_cat_layout(cref):
    g = torch.Generator().manual_seed(74)
    x = torch.randn(2, 5, 16, generator=g).to(torch.float16)
    st = torch.randn(2, 3, 16, generator=g).to(torch.float16)
    a = torch.rand(16, generator=g) + 0.5
    y = cref.snake_cat(x, st, a, 1 / a)
    assert y.shape == (2, 8, 16) and torch.equal(y[:, :3], st)
    want = (x.double() + (1 / a).double() * torch.sin(x.double() * a.double()) ** 2).to(torch.float16)
    assert ((y[:, 3:].double() - want.double()).abs() <= 2 ** -10 * want.double().abs().clamp(min=1)).all()
    assert torch.equal(cref.snake_cat(x, None, None, None), x)


@pytest.mark.parametrize("C,taps,dil,T", [(16, 7, 3, 20), (32, 3, 1, 5), (96, 7, 9, 40)])
def test_ru_fused_is_the_two_conv_unit_when_the_second_snake_is_identity(cref, C, taps, dil, T):
    """ib2 = 0: snake2 is the identity, so the fused unit's fp32 h rounds to fp16 exactly where conv_cl's
    output would: ru_fused must equal snake_cat -> conv_cl (k taps, b1) -> conv_cl (1x1, b2, + x) bit for bit."""
    g = torch.Generator().manual_seed(C + taps)
    B, ctx = 3, (taps - 1) * dil
    x = torch.randn(B, T, C, generator=g).half()
    st = torch.randn(B, ctx, C, generator=g).half()
    a1, a2 = torch.rand(C, generator=g) + 0.5, torch.rand(C, generator=g) + 0.5
    ib1 = 1.0 / (a1 + 1e-9)
    w1 = (torch.randn(taps, C, C, generator=g) / (taps * C) ** 0.5).half()
    w2 = (torch.randn(C, C, generator=g) / C ** 0.5).half()
    b1, b2 = torch.randn(C, generator=g).half(), torch.randn(C, generator=g).half()
    got = cref.ru_fused(x, st, a1, ib1, w1, b1, a2, torch.zeros(C), w2, b2, taps, dil)
    xin = cref.snake_cat(x, st, a1, ib1)
    h = cref.conv_cl(xin, w1.unsqueeze(0), b1, T, taps, dil, 1, C)
    want = cref.conv_cl(h, w2.view(1, 1, C, C), b2, T, 1, 1, 1, C, res=x)
    assert torch.equal(got, want)


def test_ru_fused_against_float64_loop(cref):
    """With the second snake: a float64 loop over rows, taps and channels (the state rows for t + j dil < ctx,
    the activated input after), the snake on fp32-exact h, one fp16 rounding of h', then the 1x1, b2 and x.
    Within one fp16 ulp (fp32 vs float64 sums may flip a rounding of h')."""
    g = torch.Generator().manual_seed(7)
    B, T, C, taps, dil = 2, 6, 16, 3, 2
    ctx = (taps - 1) * dil
    x = torch.randn(B, T, C, generator=g).half()
    st = torch.randn(B, ctx, C, generator=g).half()
    a1, a2 = torch.rand(C, generator=g) + 0.5, torch.rand(C, generator=g) + 0.5
    ib1, ib2 = 1.0 / (a1 + 1e-9), 1.0 / (a2 + 1e-9)
    w1 = (torch.randn(taps, C, C, generator=g) / (taps * C) ** 0.5).half()
    w2 = (torch.randn(C, C, generator=g) / C ** 0.5).half()
    b1, b2 = torch.randn(C, generator=g).half(), torch.randn(C, generator=g).half()
    got = cref.ru_fused(x, st, a1, ib1, w1, b1, a2, ib2, w2, b2, taps, dil).double()
    xd = x.double()
    sx = (xd + ib1.double() * torch.sin(a1.double() * xd) ** 2).half().double()   # snake1, one fp16 rounding
    want = torch.empty(B, T, C, dtype=torch.float64)
    for b in range(B):
        for t in range(T):
            h = b1.double().clone()
            for j in range(taps):
                r = t + j * dil - ctx
                row = st[b, ctx + r].double() if r < 0 else sx[b, r]
                h += row @ w1[j].double()
            hs = (h + ib2.double() * torch.sin(a2.double() * h) ** 2).half().double()
            want[b, t] = hs @ w2.double() + b2.double() + xd[b, t]
    err = (got - want).abs()
    assert (err <= want.abs() * 2 ** -9 + 2e-3).all(), err.max().item()


def test_vocoder_pack_conv_against_torch_conv():
    """The product's weight packing (vocoder.pack_conv, fast_engine.py:186-206) under the oracle's conv_cl
    equals torch's conv1d / conv_transpose1d of the module weights (conv_ref._conv_fc: causal zero context,
    right-cropped transposed conv) -- a wrong tap order, phase or transpose fails it."""
    import importlib
    voc = importlib.import_module("audio8-turbo-engine_amd.vocoder")
    from oracle import conv_ref
    g = torch.Generator().manual_seed(5)
    B, T, Cin, Cout = 2, 6, 16, 24
    x = torch.randn(B, T, Cin, generator=g).to(torch.float16)
    for trans, s, K, dil in ((False, 1, 7, 3), (False, 1, 1, 1), (True, 4, 8, 1), (True, 2, 4, 1)):
        w = torch.randn(Cin, Cout, K, generator=g) if trans else torch.randn(Cout, Cin, K, generator=g)
        b = torch.randn(Cout, generator=g)
        W, taps, ph = voc.pack_conv(w, trans, s)
        assert W.shape == (ph, taps, Cin, max(16, Cout))
        ctx = 1 if trans else (K - 1) * dil
        xin = torch.cat([torch.zeros(B, ctx, Cin, dtype=torch.float16), x], 1)
        got = conv_ref.conv_cl(xin, W, b.to(torch.float16), T, taps, dil if not trans else 1, ph, Cout)
        want = conv_ref._conv_fc(x.transpose(1, 2).double(), w, b, dil=dil, trans=trans, stride=s).transpose(1, 2)
        assert got.shape == want.shape
        err = (got.double() - want).abs()
        assert (err <= want.abs() * 2 ** -10 + 1e-3).all(), (trans, K, err.max())


def _structured_decoder(cin, ch, rates, k, dils, c):
    """decoder_weights-shaped weights under which the decoder is a known linear filter on channel 0: every snake
    the identity (alpha 1e-6: x + sin(ax)^2 / a moves a dyadic fp16 value by less than half an ulp), conv_in
    and the final conv the current tap of channel 0, each transposed conv a sample repeat (taps 0 .. s-1 of
    channel i -> i), each residual unit x + c * x(t - (k - 1) dil) (its k-conv the oldest tap, its 1x1 conv
    c times the identity)."""
    def eye_tap(co, ci, kk, tap):
        w = torch.zeros(co, ci, kk)
        for i in range(min(co, ci)):
            w[i, i, tap] = 1.0
        return w

    alpha = lambda C: torch.full((C,), 1e-6)
    wts = {"conv_in": (eye_tap(ch, cin, k, k - 1), torch.zeros(ch)), "blocks": []}
    C = ch
    for s in rates:
        tw = torch.zeros(C, C // 2, 2 * s)
        for i in range(C // 2):
            tw[i, i, :s] = 1.0
        a0 = alpha(C)
        C //= 2
        units = [(alpha(C), eye_tap(C, C, k, 0), torch.zeros(C), d, alpha(C), c * eye_tap(C, C, 1, 0), torch.zeros(C))
                 for d in dils]
        wts["blocks"].append((a0, tw, torch.zeros(C), s, units))
    wts["final"] = (alpha(C), eye_tap(1, C, k, k - 1), torch.zeros(1))
    return wts


def test_decoder_composition_closed_form():
    """The oracle decoder's composition (fast_engine.py:276-310: conv_in, per block snake + causal transposed conv
    + residual units, snake, conv_out, tanh) against the closed-form impulse response of the structured weights
    above: an impulse of height h at input time t0 leaves the transposed convs as a box of length s, each unit of
    dilation d at a block's rate multiplies the z-transform by (1 + c z^-(k-1) d) in that rate's samples, later
    blocks repeat every sample s times. A wrong block order, dilation, crop side, tap order or a non-causal
    shift moves or reweights the response."""
    from oracle import conv_ref
    cin, ch, rates, k, dils, c, T = 2, 8, (2, 4), 3, (1, 2), 0.5, 5
    wts = _structured_decoder(cin, ch, rates, k, dils, c)
    for t0, h in ((0, 0.25), (2, -0.375), (4, 0.5)):
        x = torch.zeros(1, T, cin, dtype=torch.float64)
        x[0, t0, 0] = h
        x[0, t0, 1] = 0.75  # channel 1 never reaches the output (the final conv reads channel 0)
        got = conv_ref.decoder(wts, x)[0].double()
        # closed form: the response as a dict time -> value, refined block by block
        resp = {t0: h}
        for bi, s in enumerate(rates):
            resp = {t * s + j: v for t, v in resp.items() for j in range(s)}  # repeat (box of length s)
            for d in dils:  # x + c x(t - (k - 1) d), in order
                D = (k - 1) * d
                nxt = dict(resp)
                for t, v in resp.items():
                    nxt[t + D] = nxt.get(t + D, 0.0) + c * v
                resp = nxt
        up = int(np.prod(rates))
        want = torch.zeros(T * up, dtype=torch.float64)
        for t, v in resp.items():
            if t < T * up:
                want[t] = v
        assert got.shape == want.shape
        assert torch.allclose(got, torch.tanh(want), rtol=0, atol=1e-12), (t0, (got - torch.tanh(want)).abs().max())


def test_decoder_is_causal_in_its_input():
    """Random weights at small sizes: changing input time t0 leaves every output sample before t0 * up
    unchanged, and changes the sample at t0 * up (the decoder streams, so a chunked run can equal the whole
    utterance)."""
    import importlib
    voc = importlib.import_module("audio8-turbo-engine_amd.vocoder")
    from oracle import conv_ref
    wts = voc.decoder_weights(cin=8, ch=16, rates=(2, 2), k=3, dils=(1, 2), seed=3)
    g = torch.Generator().manual_seed(4)
    T, up = 6, 4
    x = torch.randn(1, T, 8, generator=g).to(torch.float16).double()
    base = conv_ref.decoder(wts, x)[0]
    for t0 in (1, 3, 5):
        x2 = x.clone()
        x2[0, t0] += 1.0
        y = conv_ref.decoder(wts, x2)[0]
        assert torch.equal(y[:t0 * up], base[:t0 * up]), t0
        assert not torch.equal(y[t0 * up:], base[t0 * up:]), t0
