"""The codec window transformer's attention (reference serve/fast_engine.py:337-341, 368-387, 470-477):
the slow stack's kernels on a 128-position ring (K/V of position p at column p % 128), lens =
min(pos + 1, 128), caches that are views into one byte arena per row (non-dense row stride), frame after
frame past the ring's wrap, against the oracle's store + decode on CPU copies of the same caches."""
from __future__ import annotations

import pytest
import torch

from conftest import randn_bf16

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
HD = 64
WINDOW = 128
TOL = 2e-2


def say(msg):
    print(msg, flush=True)


def arena_views(st, b, nkv, layers, dev):
    """Per row one buffer [k0 | pad | v0 | pad | k1 | ...]: every cache is a view with row stride
    2 * layers * (nkv * WINDOW * HD + 8) elements (the reference's _arena_init layout, fast_engine.py:368-387)."""
    per = nkv * WINDOW * HD
    arena = torch.zeros(b, layers * 2 * (per + 8), dtype=BF, device=dev)
    for i in range(layers):
        o = i * 2 * (per + 8)
        st.kc[i] = arena[:, o:o + per].view(b, nkv, WINDOW, HD)
        st.vc[i] = arena[:, o + per + 8:o + 2 * per + 8].view(b, nkv, WINDOW, HD)
        assert st.kc[i].stride(0) == 2 * layers * (per + 8) and st.kc[i].stride() == st.vc[i].stride()
    return arena


@pytest.mark.parametrize("nq,nkv,fuse", [(14, 2, True), (14, 2, False), (16, 16, True), (8, 2, True),
                                         (16, 4, False)])
def test_codec_window_stream(a8, ref, dev, nq, nkv, fuse):
    say(f"case: codec window ring {WINDOW}, nq {nq} nkv {nkv}, fused {fuse}")
    g = torch.Generator().manual_seed(90 + nq + nkv + fuse)
    b, layers, T = 6, 2, 150
    W = (nq + 2 * nkv) * HD
    st = a8.AttnStack(layers, nq, nkv, HD, 10000.0, max_rows=b, cache_rows=b, cache_len=WINDOW, max_pos=4096,
                      dev=dev, nsplit_max=1, ring=WINDOW)
    arena_views(st, b, nkv, layers, dev)
    kref = [torch.zeros(b, nkv, WINDOW, HD, dtype=BF) for _ in range(layers)]
    vref = [torch.zeros(b, nkv, WINDOW, HD, dtype=BF) for _ in range(layers)]
    cos, sin = ref.rope_tables(10000.0, HD, 4096)
    bias = [randn_bf16(g, W, std=0.02) for _ in range(layers)]
    start = torch.tensor([0, 3, 100, 127, 128, 500], dtype=torch.int32)   # frames already decoded per row
    slot = torch.arange(b, dtype=torch.int32)                             # row r is slot r (rowmap off)
    checked = 0
    for t in range(T):
        pos = start + t
        lens = (pos + 1).clamp(max=WINDOW).int()
        qkv = [randn_bf16(g, b, W) for _ in range(layers)]
        outs = st.forward([x.to(dev) for x in qkv], [x.to(dev) for x in bias], pos.to(dev), slot.to(dev),
                          lens.to(dev), nsplit=1, rowmap=False, fuse=fuse)
        check = t % 37 == 0 or t == T - 1
        for i in range(layers):
            q = torch.zeros(b, nq, HD, dtype=BF)
            ref.bias_rope_store(qkv[i], bias[i], cos, sin, pos, slot, q, kref[i], vref[i], nq, nkv, HD, ring=WINDOW)
            if check:
                want = ref.decode_attention(q, kref[i], vref[i], lens)
                err = (outs[i].float().cpu() - want.float()).abs().max().item()
                assert err <= TOL, (t, i, err)
                checked += 1
    torch.cuda.synchronize()
    for i in range(layers):   # every ring column written where the oracle wrote it, bit for bit
        assert torch.equal(st.kc[i].cpu().view(torch.int16), kref[i].view(torch.int16))
        assert torch.equal(st.vc[i].cpu().view(torch.int16), vref[i].view(torch.int16))
    assert checked == 2 * ((T - 1) // 37 + 2)
