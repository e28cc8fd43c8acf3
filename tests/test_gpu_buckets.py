"""The auto schedule at the reference's tick buckets (fast_engine.py:669-670, 776): the first b slots of the C3
workload (KV 2048, GQA 14/2, hd 64), three layers of the fused store + decode captured as a HIP graph, the
reference's split count passed as the lower bound. Buckets of 64-128 slots take one workgroup per (row, kv head)
unit, 144-192 two units per workgroup. Each layer's output is compared with the CPU oracle within max-abs 2e-2,
the caches bit for bit, and a second replay bit for bit with the first."""
from __future__ import annotations

import pytest
import torch

import bench

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
LAYERS_CHECKED = 3


@pytest.fixture(scope="module")
def work(a8):
    return bench.build_workload(a8, torch, "C3", torch.device("cuda:0"))


@pytest.mark.parametrize("b", [64, 96, 128, 144, 160, 176])
def test_bucket_tick_against_oracle(a8, ref, work, b):
    w = work
    st, S = w["st"], w["S"]
    NQ, NKV, HD = bench.NQ, bench.NKV, bench.HD
    nsplit = a8.ref_nsplit(b, NKV)
    kind, shape = st.attn.schedule(b, S, nsplit, fused=True)
    units = b * NKV
    print(f"case: bucket {b} x {S}, {LAYERS_CHECKED} layers, schedule {kind} {shape}", flush=True)
    assert kind == "stream" and shape[0] * shape[1] * 64 >= S, "a whole-row launch"
    n_cu = st.attn.n_cu
    assert shape[2] == (units if units <= n_cu else -(-units // 2)), "one unit per workgroup up to the CU count"
    kc0 = [st.kc[i][:b].cpu() for i in range(LAYERS_CHECKED)]
    vc0 = [st.vc[i][:b].cpu() for i in range(LAYERS_CHECKED)]
    outs = [o[:b] for o in w["outs"][:LAYERS_CHECKED]]

    def tick():
        for i in range(LAYERS_CHECKED):
            st.layer(i, w["qkv"][i][:b], w["bias"][i], w["pos"][:b], w["slot"][:b], w["lens"][:b], w["q"][:b],
                     outs[i], nsplit=nsplit, rowmap=False, fuse=True)

    g = bench.capture(torch, tick)
    for o in outs:
        o.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    outs1 = [o.cpu() for o in outs]
    for o in outs:
        o.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    cos, sin = ref.rope_tables(10000.0, HD, S)
    pos, slot, lens = w["pos"][:b].cpu(), w["slot"][:b].cpu(), w["lens"][:b].cpu()
    worst = 0.0
    for i in range(LAYERS_CHECKED):
        assert torch.equal(outs[i].cpu(), outs1[i]), f"layer {i}: second replay differs"
        kc, vc = kc0[i], vc0[i]
        q = torch.empty(b, NQ, HD, dtype=BF)
        ref.bias_rope_store(w["qkv"][i][:b].cpu(), w["bias"][i].cpu(), cos, sin, pos, slot, q, kc, vc, NQ, NKV, HD)
        o_ref = ref.decode_attention(q, kc, vc, lens)
        assert torch.equal(st.kc[i][:b].cpu(), kc), f"layer {i}: K cache differs from the oracle's store"
        assert torch.equal(st.vc[i][:b].cpu(), vc), f"layer {i}: V cache differs from the oracle's store"
        err = (outs1[i].float() - o_ref.float()).abs().max().item()
        worst = max(worst, err)
        assert err <= 2e-2, f"layer {i}: max-abs {err} > 2e-2"
    print(f"bucket {b}: worst max-abs {worst:.3e}", flush=True)
