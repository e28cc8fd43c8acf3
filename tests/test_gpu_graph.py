"""The per-tick launch sequence (24 layers x [bias_rope_store -> split-K decode]) captured as one HIP graph
(torch.cuda.graph) and replayed: every replay matches the eager run bit for bit and the CPU oracle within
2e-2, also after the graph's input buffers are rewritten between replays. Also checks that the library
shares torch's HIP runtime."""
from __future__ import annotations

import os

import pytest
import torch

from conftest import randn_bf16

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
NQ, NKV, HD = 14, 2, 64
W = (NQ + 2 * NKV) * HD


def say(msg):
    print(msg, flush=True)


def test_library_shares_torch_runtime(a8):
    say("case: HIP runtime binding")
    path = os.path.realpath(a8.runtime_path())
    torch_lib = os.path.realpath(os.path.join(os.path.dirname(torch.__file__), "lib"))
    assert path.startswith(torch_lib), (path, torch_lib)


def _oracle_tick(ref, stack_kc, stack_vc, qkv, bias, pos, slot, lens, cos, sin):
    outs = []
    for i in range(len(qkv)):
        q = torch.empty(len(pos), NQ, HD, dtype=BF)
        ref.bias_rope_store(qkv[i], bias[i], cos, sin, pos, slot, q, stack_kc[i], stack_vc[i], NQ, NKV, HD)
        outs.append(ref.decode_attention(q, stack_kc[i], stack_vc[i], lens))
    return outs


@pytest.mark.parametrize("b,S,nsplit", [(16, 256, 6), (5, 1024, 16)])
def test_tick_graph_replay(a8, ref, dev, b, S, nsplit):
    say(f"case: 24-layer tick graph b={b} S={S}")
    L = 24
    g = torch.Generator().manual_seed(41)
    st = a8.AttnStack(L, NQ, NKV, HD, 10000.0, max_rows=max(16 * b, 64), cache_rows=b + 1, cache_len=S,
                      max_pos=S, dev=dev)
    kc0, vc0 = randn_bf16(g, L, b + 1, NKV, S, HD), randn_bf16(g, L, b + 1, NKV, S, HD)
    st.kc_all.copy_(kc0.to(dev))
    st.vc_all.copy_(vc0.to(dev))
    pos_h = torch.randint(0, S, (b,), generator=g).int()
    pos, slot, lens = pos_h.to(dev), torch.arange(b, dtype=torch.int32, device=dev), (pos_h + 1).to(dev)
    qkv = [randn_bf16(g, b, W).to(dev) for _ in range(L)]
    bias = [randn_bf16(g, W, std=0.02).to(dev) for _ in range(L)]
    q = torch.empty(b, NQ, HD, dtype=BF, device=dev)
    outs = [torch.empty(b, NQ, HD, dtype=BF, device=dev) for _ in range(L)]

    def tick():
        st.forward(qkv, bias, pos, slot, lens, nsplit=nsplit, rowmap=False, q=q, outs=outs)

    tick()
    torch.cuda.synchronize()
    eager = [o.cpu() for o in outs]
    kc_h, vc_h = list(kc0.unbind(0)), list(vc0.unbind(0))
    kc_h, vc_h = [k.clone() for k in kc_h], [v.clone() for v in vc_h]
    cos, sin = ref.rope_tables(10000.0, HD, S)
    want = _oracle_tick(ref, kc_h, vc_h, [x.cpu() for x in qkv], [x.cpu() for x in bias], pos_h,
                        torch.arange(b, dtype=torch.int32), pos_h + 1, cos, sin)
    for i in range(L):
        assert (eager[i].float() - want[i].float()).abs().max() <= 2e-2, i
    assert torch.equal(st.kc_all.cpu(), torch.stack(kc_h)) and torch.equal(st.vc_all.cpu(), torch.stack(vc_h))

    # capture (warm up on a side stream first, as the reference's capture() does)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        tick()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        tick()
    for rep in range(3):
        for o in outs:
            o.fill_(0)                                    # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i in range(L):
            assert torch.equal(outs[i].cpu(), eager[i]), (rep, i)
    # new inputs written into the captured buffers are picked up by the next replay
    for i in range(L):
        qkv[i].copy_(randn_bf16(g, b, W).to(dev))
    graph.replay()
    torch.cuda.synchronize()
    want2 = _oracle_tick(ref, kc_h, vc_h, [x.cpu() for x in qkv], [x.cpu() for x in bias], pos_h,
                         torch.arange(b, dtype=torch.int32), pos_h + 1, cos, sin)
    for i in range(L):
        assert (outs[i].cpu().float() - want2[i].float()).abs().max() <= 2e-2, i
