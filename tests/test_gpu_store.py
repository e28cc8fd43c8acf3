"""GPU parity of the fused bias + RoPE + KV store (a8_bias_rope_store through the package shim) against
the golden vectors and the CPU oracle: bit-exact for every value and every cache position."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bf16_from_bits, bits_of, golden, randn_bf16

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
NQ, NKV, HD = 14, 2, 64
W = (NQ + 2 * NKV) * HD


def say(msg):
    print(msg, flush=True)


def _run_both(a8, ref, dev, qkv, bias, cos, sin, pos, slot, kc0, vc0, ring=1 << 30, qo_shape=None, kc_view=None):
    """Store on the GPU and in the oracle from the same inputs; returns (gpu, oracle) triples (qo, kc, vc)."""
    R = qkv.shape[0]
    qo_c = torch.zeros(R, NQ, HD, dtype=BF)
    kc_c, vc_c = kc0.clone(), vc0.clone()
    ref.bias_rope_store(qkv, bias, cos, sin, pos, slot, qo_c, kc_c, vc_c, NQ, NKV, HD, ring=ring)
    qo_d = torch.zeros(R, NQ, HD, dtype=BF, device=dev)
    if kc_view is None:
        kc_d, vc_d = kc0.to(dev), vc0.to(dev)
        kv_d, vv_d = kc_d, vc_d
    else:
        kc_d, vc_d, kv_d, vv_d = kc_view(kc0, vc0)
    a8.bias_rope_store(qkv.to(dev), None if bias is None else bias.to(dev), cos.to(dev), sin.to(dev), pos.to(dev),
                       slot.to(dev), qo_d, kv_d, vv_d, NQ, NKV, HD, ring=ring)
    torch.cuda.synchronize()
    return (qo_d.cpu(), kc_d.cpu(), vc_d.cpu()), (qo_c, kc_c, vc_c)


def _assert_same(got, want):
    for g_, w_, name in zip(got, want, ("qo", "kc", "vc")):
        assert torch.equal(g_.view(torch.int16), w_.view(torch.int16)), name


def test_store_golden(a8, ref, dev):
    say("case: store golden vectors")
    z = golden("store.npz")
    sent = int(z["sentinel"])
    rows, S = int(z["rows"]), int(z["S"])
    kc = bf16_from_bits(np.full((rows, NKV, S, HD), sent, np.uint16)).to(dev)
    vc = kc.clone()
    qo = bf16_from_bits(np.full(z["qo"].shape, sent, np.uint16)).to(dev)
    a8.bias_rope_store(bf16_from_bits(z["qkv"]).to(dev), bf16_from_bits(z["bias"]).to(dev),
                       bf16_from_bits(z["cos"]).to(dev), bf16_from_bits(z["sin"]).to(dev),
                       torch.from_numpy(z["pos"]).to(dev), torch.from_numpy(z["slot"]).to(dev), qo, kc, vc, NQ, NKV, HD,
                       ring=int(z["ring"]))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits_of(qo.cpu()), z["qo"])
    np.testing.assert_array_equal(bits_of(kc.cpu()), z["kc"])
    np.testing.assert_array_equal(bits_of(vc.cpu()), z["vc"])


CONFIGS = {
    # name: (R, rows, S, positions, slots)
    "C1": (1, 2, 512, lambda g, R: torch.tensor([384]), lambda g, R: torch.tensor([0])),
    "C2": (64, 65, 4096, lambda g, R: torch.randint(127, 2048, (R,), generator=g), lambda g, R: torch.arange(R)),
    "C3": (192, 193, 2048, lambda g, R: torch.full((R,), 2047), lambda g, R: torch.arange(R)),
    "C5": (384, 192, 10, lambda g, R: torch.arange(R) % 2, lambda g, R: torch.arange(R) // 2),
}


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_store_configs(a8, ref, dev, name):
    R, rows, S, fpos, fslot = CONFIGS[name]
    say(f"case: store {name} R={R} rows={rows} S={S}")
    g = torch.Generator().manual_seed(11)
    qkv, bias = randn_bf16(g, R, W), randn_bf16(g, W, std=0.02)
    cos, sin = ref.rope_tables(10000.0, HD, max(S, 2048))
    pos, slot = fpos(g, R).int(), fslot(g, R).int()
    kc0, vc0 = randn_bf16(g, rows, NKV, S, HD), randn_bf16(g, rows, NKV, S, HD)
    got, want = _run_both(a8, ref, dev, qkv, bias, cos, sin, pos, slot, kc0, vc0)
    _assert_same(got, want)


def test_store_packed_prefill_rows(a8, ref, dev):
    """C4's store: ~14k packed rows at positions p0 + j of their request's slot."""
    say("case: store C4 packed rows")
    g = torch.Generator().manual_seed(12)
    ns = torch.randint(40, 401, (64,), generator=g).tolist()
    pos = torch.cat([300 + torch.arange(n) for n in ns]).int()
    slot = torch.cat([torch.full((n,), i) for i, n in enumerate(ns)]).int()
    R, S = len(pos), 704
    qkv, bias = randn_bf16(g, R, W), randn_bf16(g, W, std=0.02)
    cos, sin = ref.rope_tables(10000.0, HD, S)
    kc0 = torch.zeros(65, NKV, S, HD, dtype=BF)
    got, want = _run_both(a8, ref, dev, qkv, bias, cos, sin, pos, slot, kc0, kc0.clone())
    _assert_same(got, want)


def test_store_ring_no_bias_strided(a8, ref, dev):
    """Ring wrap (pos % 128), no bias, a qkv row stride wider than the row, and a non-dense cache row
    stride (the codec's byte-arena views)."""
    say("case: store ring=128, bias None, strided qkv, arena-strided cache")
    g = torch.Generator().manual_seed(13)
    R, rows, S = 40, 40, 128
    qkv_full = randn_bf16(g, R, W + 64)
    qkv = qkv_full[:, 32:32 + W]                                      # row stride W+64, 64-byte offset
    cos, sin = ref.rope_tables(10000.0, HD, 8192)
    pos = torch.randint(0, 8192, (R,), generator=g).int()
    slot = torch.randperm(rows, generator=g)[:R].int()
    kc0, vc0 = randn_bf16(g, rows, NKV, S, HD), randn_bf16(g, rows, NKV, S, HD)

    def arena(kc0, vc0):
        # one byte arena per row: [k | pad | v | pad], row stride not a multiple of the cache row
        per = NKV * S * HD
        buf = torch.zeros(rows, 2 * per + 3 * 8, dtype=BF, device=dev)
        kv = buf[:, :per].view(rows, NKV, S, HD)
        vv = buf[:, per + 8:2 * per + 8].view(rows, NKV, S, HD)
        kv.copy_(kc0.to(dev))
        vv.copy_(vc0.to(dev))
        return kv, vv, kv, vv

    got, want = _run_both(a8, ref, dev, qkv.contiguous(), None, cos, sin, pos, slot, kc0, vc0, ring=128)
    _assert_same(got, want)
    # same through the strided views (the shim passes the row stride through; vc shares kc's strides)
    qo_d = torch.zeros(R, NQ, HD, dtype=BF, device=dev)
    kv, vv, _, _ = arena(kc0, vc0)
    assert kv.stride() == vv.stride() and kv.stride(0) != NKV * S * HD
    a8.bias_rope_store(qkv_full.to(dev)[:, 32:32 + W], None, cos.to(dev),
                       sin.to(dev), pos.to(dev), slot.to(dev), qo_d, kv, vv, NQ, NKV, HD, ring=128)
    torch.cuda.synchronize()
    _assert_same((qo_d.cpu(), kv.cpu(), vv.cpu()), want)


def test_store_out_of_range_rows_write_nothing(a8, ref, dev):
    """Rows whose position is outside the tables or whose slot / ring position is outside the cache store
    nothing (kernel-side bounds checks); in-range rows are unaffected."""
    say("case: store out-of-range rows")
    g = torch.Generator().manual_seed(14)
    R, rows, S = 6, 3, 64
    qkv = randn_bf16(g, R, W)
    cos, sin = ref.rope_tables(10000.0, HD, 100)
    pos = torch.tensor([5, 100, -1, 70, 7, 8], dtype=torch.int32)     # 100, -1: off the table; 70 >= S
    slot = torch.tensor([0, 0, 1, 1, 3, 2], dtype=torch.int32)        # 3 >= rows
    kc0 = randn_bf16(g, rows, NKV, S, HD)
    good = torch.tensor([0, 5])
    qo_c = torch.zeros(R, NQ, HD, dtype=BF)
    kc_c, vc_c = kc0.clone(), kc0.clone()
    ref.bias_rope_store(qkv[good], None, cos, sin, pos[good], slot[good], qo_c[:2], kc_c, vc_c, NQ, NKV, HD)
    qo_d = torch.zeros(R, NQ, HD, dtype=BF, device=dev)
    kc_d, vc_d = kc0.to(dev), kc0.to(dev)
    a8.bias_rope_store(qkv.to(dev), None, cos.to(dev), sin.to(dev), pos.to(dev), slot.to(dev), qo_d, kc_d, vc_d,
                       NQ, NKV, HD)
    torch.cuda.synchronize()
    assert torch.equal(kc_d.cpu(), kc_c) and torch.equal(vc_d.cpu(), vc_c)
    assert torch.equal(qo_d.cpu()[good], qo_c[:2])
    assert not qo_d.cpu()[1:3].view(torch.int16).any()               # off-table rows: q not written
