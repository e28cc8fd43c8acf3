"""Host-side logic of the package on the CPU: argument validation of the operator shims (mirroring the
reference's asserts / type errors), the plan builders and the caller-side helpers."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from conftest import randn_bf16

BF = torch.bfloat16


def test_helpers_match_oracle(a8, ref):
    for n in (1, 10, 2048):
        c0, s0 = a8.rope_tables(10000.0, 64, n, "cpu")
        c1, s1 = ref.rope_tables(10000.0, 64, n)
        assert torch.equal(c0, c1) and torch.equal(s0, s1)
    w = torch.randn(1152, 9, dtype=torch.float64)
    assert torch.equal(a8.permute_qk(w, 14, 2, 64), ref.permute_qk(w, 14, 2, 64))
    for b in (1, 3, 8, 16, 33, 64, 127, 192):
        assert a8.ref_nsplit(b, 2) == ref.ref_nsplit(b, 2)


def _heaviest_first_of(got, want):
    """got (q0, n, slot, pos0 columns) lists the blocks of want in order of key count pos0 + n, largest
    first, ties in want's order."""
    got, want = list(zip(*[list(map(int, c)) for c in got])), list(zip(*[list(map(int, c)) for c in want]))
    assert sorted(got) == sorted(want)
    assert got == sorted(want, key=lambda b: -(b[3] + b[1]))
    keys = [b[3] + b[1] for b in got]
    assert keys == sorted(keys, reverse=True)


def test_prefill_plan_matches_oracle(a8, ref):
    """The plan's q0, n, slot, pos0 are the reference's blocks in its order (exact int equality); the
    dispatch copy holds the same blocks heaviest first."""
    r0s, ns, slots, p0s = [0, 70, 75], [70, 5, 200], [3, 1, 0], [300, 0, 64]
    p = a8.PrefillPlan(r0s, ns, slots, p0s, "cpu")
    want = ref.prefill_plan(r0s, ns, slots, p0s)
    assert p.nblk == len(want[0]) == 2 + 1 + 4
    assert all(t.dtype == torch.int32 for t in (p.q0, p.n, p.slot, p.pos0))
    assert [p.q0.tolist(), p.n.tolist(), p.slot.tolist(), p.pos0.tolist()] == [list(map(int, c)) for c in want]
    d = p.dispatch
    _heaviest_first_of((d.q0.tolist(), d.n.tolist(), d.slot.tolist(), d.pos0.tolist()), want)
    assert d.pos0.tolist()[:2] == [300 + 64, 300]  # request 0's blocks (keys 370 and 364) lead
    assert a8.PrefillPlan.BM == 64
    assert a8.PrefillPlan([], [], [], [], "cpu").nblk == 0


def test_prefill_meta_matches_oracle(a8, ref):
    """The buffer's first nine fields equal the reference's graph-mode plan (fast_engine.py:837-853) int for
    int; the four dispatch fields hold its blocks heaviest first, then the same padding blocks."""
    meta = a8.PrefillMeta(2048, 64, 192, "cpu")
    for slots, ns, starts, nt in (([], [], [], 2048), ([5, 9], [300, 64], [300, 300], 512),
                                  (list(range(64)), [1] * 64, list(range(64)), 64)):
        h = meta.host(nt, slots, ns, starts)
        w = ref.pf_meta_host(nt, slots, ns, starts, 2048, 64, 192)
        o = meta.off
        np.testing.assert_array_equal(h[:o[9]], w)
        nb = int((w[o[3]:o[4]] > 0).sum())
        cols = [lambda m, i=i: m[o[i]:o[i] + nb] for i in (2, 3, 4, 5)]
        dcols = [lambda m, i=i: m[o[i]:o[i] + nb] for i in (9, 10, 11, 12)]
        _heaviest_first_of([c(h) for c in dcols], [c(w) for c in cols])
        for i, j in zip((9, 10, 11, 12), (2, 3, 4, 5)):  # padding blocks as the reference's
            np.testing.assert_array_equal(h[o[i] + nb:o[i + 1]], w[o[j] + nb:o[j + 1]])
    meta.load(512, [5, 9], [300, 64], [300, 300])
    plan = meta.plan(512)
    assert plan.nblk == 512 // 64 + 64 and plan.BM == 64
    assert plan.n[:6].tolist() == [64, 64, 64, 64, 44, 64] and (plan.n[6:] == 0).all()
    assert plan.pos0[:6].tolist() == [300, 364, 428, 492, 556, 300]
    assert plan.dispatch.n[:6].tolist() == [44, 64, 64, 64, 64, 64] and (plan.dispatch.n[6:] == 0).all()
    assert plan.dispatch.pos0[:6].tolist() == [556, 492, 428, 364, 300, 300]
    assert (plan.slot[6:] == 192).all() and (plan.dispatch.slot[6:] == 192).all()


def _store_inputs(dev="cpu"):
    g = torch.Generator().manual_seed(0)
    return dict(qkv=randn_bf16(g, 2, 1152), bias=randn_bf16(g, 1152), cos_tab=torch.zeros(16, 64, dtype=BF),
                sin_tab=torch.zeros(16, 64, dtype=BF), pos=torch.zeros(2, dtype=torch.int32),
                slot=torch.zeros(2, dtype=torch.int32), qo=torch.empty(2, 14, 64, dtype=BF),
                kc=torch.zeros(1, 2, 16, 64, dtype=BF), vc=torch.zeros(1, 2, 16, 64, dtype=BF), nq=14, nkv=2, hd=64)


def test_store_shim_validation(a8):
    a = _store_inputs()
    with pytest.raises(ValueError, match="HIP device"):
        a8.bias_rope_store(**a)
    with pytest.raises(TypeError, match="bfloat16"):
        a8.bias_rope_store(**{**a, "qkv": a["qkv"].float()})
    with pytest.raises(TypeError, match="int32"):
        a8.bias_rope_store(**{**a, "pos": a["pos"].long()})


def test_decode_shim_validation(a8):
    att = a8.DecodeAttention(8, 14, 2, 64, 16, "cpu")
    assert att.group == 7 and att.gp == 16 and att.scale == 0.125
    assert att.acc_flat.numel() == 8 * 14 * 64 and att.ml_flat.numel() == 8 * 14 * 2
    q = torch.zeros(3, 14, 64, dtype=BF)
    kc = torch.zeros(3, 2, 8, 64, dtype=BF)
    lens = torch.ones(3, dtype=torch.int32)
    with pytest.raises(AssertionError):                     # fast_kernels.py:276: b * nsplit <= cap
        att(q, kc, kc, lens, q, nsplit=3)
    # an fp32 query takes its own entry point (validated the same way: device tensors only)
    with pytest.raises(ValueError, match="HIP device"):
        att(q.float(), kc, kc, lens, q, nsplit=1)
    with pytest.raises(TypeError):                          # out must be bf16 or fp32
        att(q.float(), kc, kc, lens, q.half(), nsplit=1)
    with pytest.raises(TypeError):                          # q must be bf16 or fp32
        att(q.half(), kc, kc, lens, q, nsplit=1)
    with pytest.raises(NotImplementedError):
        att(q, kc, kc, lens, q, nsplit=1, bn=32)
    with pytest.raises(ValueError, match="HIP device"):
        att(q, kc, kc, lens, q, nsplit=1)


def test_prefill_shim_validation(a8):
    q = torch.zeros(4, 14, 64, dtype=BF)
    kc = torch.zeros(1, 2, 8, 64, dtype=BF)
    plan = SimpleNamespace(q0=torch.zeros(1, dtype=torch.int32), n=torch.ones(1, dtype=torch.int32),
                           slot=torch.zeros(1, dtype=torch.int32), pos0=torch.zeros(1, dtype=torch.int32), nblk=1, BM=64)
    with pytest.raises(ValueError, match="group"):
        a8.prefill_attention(q, kc, kc, plan, q, 5)
    with pytest.raises(ValueError, match="HIP device"):
        a8.prefill_attention(q, kc, kc, plan, q, 7)


def test_package_has_no_cpu_fallback():
    """The product package never imports the oracle or computes attention with torch ops. The one torch
    GEMM is the slow stack's projection `mm` (the reference's own default, a library GEMM), outside the
    attention path (GemmDispatch's library choice is the same GEMM)."""
    import os
    import re
    from conftest import ROOT
    pkg = os.path.join(ROOT, "audio8-turbo-engine_amd")
    for f in os.listdir(pkg):
        if f.endswith(".py"):
            src = open(os.path.join(pkg, f)).read()
            assert not re.search(r"\boracle\b", src.replace("oracle (", "")), f
            if f in ("slow_stack.py", "fast_kernels.py"):
                # the projections' library GEMM (the slow stack's default `mm`, GemmDispatch's library choice)
                # is the only torch product allowed, and only in these two files
                src = re.sub(r"torch\.matmul\(x, w\.t\(\)(, out=y)?\)", "", src)
            for call in ("softmax(", "scaled_dot_product", "matmul(", "einsum(", "bmm(", ".exp("):
                assert call not in src, (f, call)
