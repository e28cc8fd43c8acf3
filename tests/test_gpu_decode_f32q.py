"""fp32-query decode (the reference's PREC = "ieee" branch, fast_kernels.py:279) through DecodeAttention ->
a8_decode_attn_f32q, against the oracle's decode_attention on the same fp32 q (oracle/attn_ref.py; its fp32-q
path is pinned by tests/test_oracle.py::test_decode_fp32_query_against_float64): ragged lengths, the edges
(0 -> NaN like the reference, 1, tile multiples, past the cache), a row map, head_dim 128, bf16 and fp32
outputs. Bar: max-abs <= 2e-2 (the weights are rounded to bf16 for P.V, relative to a running maximum that
depends on the key order), and the fp32 output within 1e-2 of the oracle's fp32 output."""
from __future__ import annotations

import pytest
import torch

from conftest import randn_bf16

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("case", ["C1", "ragged", "edges", "rowmap", "hd128"])
@pytest.mark.parametrize("out_dtype", [BF, torch.float32])
def test_decode_fp32_query(a8, ref, dev, case, out_dtype):
    say(f"case: fp32-q decode {case} out {out_dtype}")
    g = torch.Generator().manual_seed(90 + len(case))
    nq, nkv, hd = 14, 2, 128 if case == "hd128" else 64
    rowmap = None
    if case == "C1":
        b, rows, S, lens = 1, 1, 512, torch.tensor([385])
    elif case == "ragged":
        b, rows, S = 24, 24, 1024
        lens = torch.randint(1, 1025, (b,), generator=g)
    elif case == "edges":
        b, rows, S = 8, 8, 200
        lens = torch.tensor([0, 1, 63, 64, 65, 128, 200, 999])
    elif case == "rowmap":
        b, rows, S = 12, 6, 300
        lens = torch.randint(1, 301, (b,), generator=g)
        rowmap = (torch.arange(b) // 2).int()
    else:
        b, rows, S = 10, 10, 700
        lens = torch.randint(1, 701, (b,), generator=g)
    lens = lens.int()
    q = torch.randn(b, nq, hd, generator=g)
    kc, vc = randn_bf16(g, rows, nkv, S, hd), randn_bf16(g, rows, nkv, S, hd)
    want = ref.decode_attention(q, kc, vc, lens.clamp(max=S), nsplit=1, rowmap=rowmap, out_dtype=out_dtype)
    att = a8.DecodeAttention(max(16 * b, 64), nq, nkv, hd, 16, dev)
    out = torch.full((b, nq, hd), 3.0, dtype=out_dtype, device=dev)
    att(q.to(dev), kc.to(dev), vc.to(dev), lens.to(dev), out, nsplit=4,
        rowmap=None if rowmap is None else rowmap.to(dev))
    torch.cuda.synchronize()
    got = out.cpu()
    nan_rows = (lens == 0).nonzero().flatten().tolist()
    for r in nan_rows:
        assert torch.isnan(got[r].float()).all() and torch.isnan(want[r].float()).all()
    keep = [r for r in range(b) if r not in nan_rows]
    err = (got[keep].float() - want[keep].float()).abs().max().item()
    say(f"  max-abs {err:.3e}")
    assert err <= (1e-2 if out_dtype == torch.float32 else 2e-2)


def test_decode_fp32_query_differs_from_rounded_query(a8, ref, dev):
    """The fp32 query is used as is, not rounded to bf16 first: against the oracle with q rounded to bf16, the
    kernel's output moves by far more than its own error against the fp32-q oracle (a query scaled so that
    its rounding matters)."""
    say("case: fp32-q decode keeps the query's low bits")
    g = torch.Generator().manual_seed(77)
    b, nq, nkv, hd, S = 4, 14, 2, 64, 256
    q = torch.randn(b, nq, hd, generator=g) * 8.0
    kc, vc = randn_bf16(g, b, nkv, S, hd), randn_bf16(g, b, nkv, S, hd)
    lens = torch.full((b,), S, dtype=torch.int32)
    att = a8.DecodeAttention(64, nq, nkv, hd, 16, dev)
    out = torch.empty(b, nq, hd, dtype=torch.float32, device=dev)
    att(q.to(dev), kc.to(dev), vc.to(dev), lens.to(dev), out)
    torch.cuda.synchronize()
    exact = ref.decode_attention(q, kc, vc, lens, out_dtype=torch.float32)
    rounded = ref.decode_attention(q.to(BF), kc, vc, lens, out_dtype=torch.float32)
    e_exact = (out.cpu() - exact).abs().max().item()
    e_round = (out.cpu() - rounded).abs().max().item()
    say(f"  vs fp32-q oracle {e_exact:.3e}, vs bf16-q oracle {e_round:.3e}")
    assert e_exact < 0.25 * e_round
