"""The benchmark's C2 tick, checked in full: 64 slots with ragged lengths U[128, 2048] over a 4096-position cache,
GQA 14/2, hd 64, 24 layers, built by bench.build_workload; per layer the fused store + split decode launch and the
combine, at the launch shape the engine's chooser takes, captured as a HIP graph and replayed. Every layer's output
is compared with the CPU oracle (store, then textbook decode) within the north-star tolerance (max-abs 2e-2), every
layer's K / V cache bit for bit, and a second replay bit for bit with the first."""
from __future__ import annotations

import pytest
import torch

import bench

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def say(msg):
    print(msg, flush=True)


def test_bench_tick_c2_against_oracle(a8, ref):
    dev = torch.device("cuda:0")
    w = bench.build_workload(a8, torch, "C2", dev)
    st, b, S = w["st"], w["b"], w["S"]
    L, NQ, NKV, HD = bench.LAYERS, bench.NQ, bench.NKV, bench.HD
    nsplit = a8.ref_nsplit(b, NKV)
    kind, shape = st.attn.schedule(b, S, nsplit, fused=True)
    say(f"case: C2 tick {b} rows, lengths {int(w['lens_h'].min())}..{int(w['lens_h'].max())}, cache {S}, "
        f"{L} layers, schedule {kind} {shape}")
    assert kind == "split" and shape[0] > 1, "the split launch with its combine"
    kc0 = [st.kc[i].cpu() for i in range(L)]
    vc0 = [st.vc[i].cpu() for i in range(L)]

    def tick():
        st.forward(w["qkv"], w["bias"], w["pos"], w["slot"], w["lens"], nsplit=nsplit, rowmap=False, q=w["q"],
                   outs=w["outs"], fuse=True)

    g = bench.capture(torch, tick)
    for o in w["outs"]:
        o.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    outs1 = [o.cpu() for o in w["outs"]]
    for o in w["outs"]:
        o.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    for i in range(L):
        assert torch.equal(w["outs"][i].cpu(), outs1[i]), f"layer {i}: second replay differs"

    cos, sin = ref.rope_tables(10000.0, HD, S)
    pos, slot, lens = w["pos"].cpu(), w["slot"].cpu(), w["lens"].cpu()
    worst = 0.0
    for i in range(L):
        kc, vc = kc0[i], vc0[i]
        q = torch.empty(b, NQ, HD, dtype=BF)
        ref.bias_rope_store(w["qkv"][i].cpu(), w["bias"][i].cpu(), cos, sin, pos, slot, q, kc, vc, NQ, NKV, HD)
        o_ref = ref.decode_attention(q, kc, vc, lens)
        assert torch.equal(st.kc[i].cpu(), kc), f"layer {i}: K cache differs from the oracle's store"
        assert torch.equal(st.vc[i].cpu(), vc), f"layer {i}: V cache differs from the oracle's store"
        err = (outs1[i].float() - o_ref.float()).abs().max().item()
        worst = max(worst, err)
        assert err <= 2e-2, f"layer {i}: max-abs {err} > 2e-2"
    say(f"C2 tick: 24 layers, worst max-abs {worst:.3e}")
