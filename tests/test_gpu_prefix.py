"""The admission copy of a cached voice prefix's K/V into slots (a8_prefix_copy) against the reference's own
index-puts, kc_all[:, idx, :, :Lp] = k.unsqueeze(1) (serve/fast_engine.py:1098-1103), run by torch on the
same GPU tensors: bit for bit."""
from __future__ import annotations

import pytest
import torch

from conftest import randn_bf16

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def say(msg):
    print(msg, flush=True)


def _case(g, dev, layers, rows, nkv, S):
    kc_all = randn_bf16(g, layers, rows, nkv, S, 64).to(dev)
    vc_all = randn_bf16(g, layers, rows, nkv, S, 64).to(dev)
    return kc_all, vc_all


@pytest.mark.parametrize("layers,rows,nkv,S,Lp,nslots", [(24, 70, 2, 704, 300, 16), (3, 9, 2, 128, 1, 9),
                                                          (2, 5, 4, 256, 129, 3), (4, 20, 2, 2048, 2048, 5)])
def test_prefix_copy_matches_index_put(a8, dev, layers, rows, nkv, S, Lp, nslots):
    say(f"case: prefix copy layers {layers} rows {rows} nkv {nkv} S {S} Lp {Lp} slots {nslots}")
    g = torch.Generator().manual_seed(layers + rows + Lp)
    kc_all, vc_all = _case(g, dev, layers, rows, nkv, S)
    k = randn_bf16(g, layers, nkv, Lp, 64).to(dev)
    v = randn_bf16(g, layers, nkv, Lp, 64).to(dev)
    slots = torch.randperm(rows, generator=g)[:nslots].tolist()
    want_k, want_v = kc_all.clone(), vc_all.clone()
    idx = torch.tensor(slots, dtype=torch.long, device=dev)
    want_k[:, idx, :, :Lp] = k.unsqueeze(1)
    want_v[:, idx, :, :Lp] = v.unsqueeze(1)
    a8.prefix_copy(k, v, kc_all, vc_all, torch.tensor(slots, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    assert torch.equal(kc_all.view(torch.int16), want_k.view(torch.int16))
    assert torch.equal(vc_all.view(torch.int16), want_v.view(torch.int16))


def test_prefix_copy_views_duplicates_and_bad_slots(a8, dev):
    """The prefix taken as a view of the scratch row (as _prefix_kv slices it before cloning), a slot listed
    twice, slots outside the cache (skipped), a list of slots (uploaded by the shim), and a cache that is a
    view with a wider row stride."""
    say("case: prefix copy from a view, duplicate and invalid slots, strided cache")
    g = torch.Generator().manual_seed(5)
    layers, rows, nkv, S, Lp = 4, 12, 2, 320, 300
    big_k, big_v = _case(g, dev, layers, rows + 2, nkv, S + 64)
    kc_all, vc_all = big_k[:, 1:rows + 1, :, 32:32 + S], big_v[:, 1:rows + 1, :, 32:32 + S]
    scratch = rows - 1
    k, v = kc_all[:, scratch, :, :Lp], vc_all[:, scratch, :, :Lp]          # views: strides of the cache
    k_src, v_src = k.clone(), v.clone()
    before_k, before_v = big_k.clone(), big_v.clone()
    slots = [3, 0, 3, -1, rows, 7]
    a8.prefix_copy(k, v, kc_all, vc_all, slots)
    torch.cuda.synchronize()
    want_k, want_v = before_k.clone(), before_v.clone()
    wk, wv = want_k[:, 1:rows + 1, :, 32:32 + S], want_v[:, 1:rows + 1, :, 32:32 + S]
    idx = torch.tensor([3, 0, 7], dtype=torch.long, device=dev)
    wk[:, idx, :, :Lp] = k_src.unsqueeze(1)
    wv[:, idx, :, :Lp] = v_src.unsqueeze(1)
    assert torch.equal(big_k.view(torch.int16), want_k.view(torch.int16))   # nothing else touched
    assert torch.equal(big_v.view(torch.int16), want_v.view(torch.int16))
    a8.prefix_copy(k, v, kc_all, vc_all, [])                                 # no slots: nothing launched
