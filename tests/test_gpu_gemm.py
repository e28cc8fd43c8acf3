"""GPU parity of the small-M GEMM (a8_gemm_small through gemm_small / GemmDispatch) against a float64 product
(the semantics of the oracle's linear, oracle/layer_ref.py: fp32 accumulation of bf16 products, bf16 out):
the slow-AR projections at the decode tick's 192 rows and every split count, ragged M and N, and a
GemmDispatch tuned then captured in a graph. Bar: within 2 bf16 ulps of a float64 product (relative to the
output's scale), splits deterministic (two runs bit for bit)."""
from __future__ import annotations

import pytest
import torch

from conftest import randn_bf16

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def say(msg):
    print(msg, flush=True)


def _check(got, x, w):
    want = x.double() @ w.double().T
    err = (got.double().cpu() - want).abs()
    # bf16 rounding of the result plus fp32 accumulation-order noise
    tol = 2 * 2.0 ** -8 * want.abs() + 1e-3 * want.abs().max()
    assert (err <= tol).all(), f"max err {err.max().item():.3e}"
    return err.max().item()


# the slow AR's projections at 192 rows: qkv (1152 x 896), o (896 x 896), w13 (9728 x 896), w2 (896 x 4864)
@pytest.mark.parametrize("N,K", [(1152, 896), (896, 896), (9728, 896), (896, 4864)])
@pytest.mark.parametrize("splits,mblocks", [(1, 1), (4, 1), (16, 1), (1, 3), (3, 6), (2, 2)])
def test_gemm_slow_ar_shapes(a8, dev, N, K, splits, mblocks):
    say(f"case: gemm M=192 N={N} K={K} splits={splits} mblocks={mblocks}")
    g = torch.Generator().manual_seed(N + K)
    x, w = randn_bf16(g, 192, K), (randn_bf16(g, N, K) / K ** 0.5).to(BF)
    xd, wd = x.to(dev), w.to(dev)
    ws = torch.zeros(a8.gemm_ws_bytes(192, N, 16), dtype=torch.uint8, device=dev)
    a = a8.gemm_small(xd, wd, splits=splits, ws=ws, mblocks=mblocks)
    b = a8.gemm_small(xd, wd, splits=splits, ws=ws, mblocks=mblocks)
    torch.cuda.synchronize()
    assert torch.equal(a, b), "two runs differ"
    err = _check(a, x, w)
    say(f"  max err {err:.3e}")
    if splits == 1 and mblocks > 1:  # row blocks do not change a single product
        assert torch.equal(a, a8.gemm_small(xd, wd))
    assert (ws[:4096] == 0).all(), "tile counters not back at zero"


@pytest.mark.parametrize("M,N,K,splits,mblocks", [(1, 8, 64, 1, 1), (5, 72, 128, 2, 1), (17, 136, 640, 3, 1),
                                                  (100, 200, 1024, 5, 3), (191, 1000, 896, 7, 2),
                                                  (33, 64, 64, 4, 6), (150, 96, 192, 1, 5), (65, 24, 128, 2, 3)])
def test_gemm_ragged(a8, dev, M, N, K, splits, mblocks):
    """M and N not multiples of the tiles (rows past M / N read as zeros and are not stored), splits above the
    chunk count, row blocks that do not divide M, and strided x / out views."""
    say(f"case: gemm ragged M={M} N={N} K={K} splits={splits} mblocks={mblocks}")
    g = torch.Generator().manual_seed(M * 7 + N)
    xb = randn_bf16(g, M, K + 64)
    x = xb[:, 32:32 + K]                     # row stride K + 64, 64-byte offset
    w = randn_bf16(g, N, K)
    outb = torch.full((M, N + 16), 5.0, dtype=BF, device=dev)
    out = outb[:, 8:8 + N]
    ws = torch.zeros(a8.gemm_ws_bytes(M, N, 8) + 64, dtype=torch.uint8, device=dev)
    a8.gemm_small(xb.to(dev)[:, 32:32 + K], w.to(dev), out=out, splits=splits, ws=ws, mblocks=mblocks)
    torch.cuda.synchronize()
    _check(out, x, w)
    assert (outb[:, :8].float() == 5.0).all() and (outb[:, 8 + N:].float() == 5.0).all()


def test_gemm_workspace_shared_across_shapes(a8, dev):
    """One zeroed workspace through calls of different shapes, split counts and row blocks (the counters sit
    at its start for every shape and are left at zero): each result right, the counters zero at the end."""
    say("case: gemm one workspace, several shapes")
    g = torch.Generator().manual_seed(11)
    ws = torch.zeros(a8.gemm_ws_bytes(192, 9728, 7), dtype=torch.uint8, device=dev)
    for M, N, K, sp, mb in [(192, 896, 4864, 7, 3), (192, 9728, 896, 3, 1), (64, 1152, 896, 2, 2),
                            (192, 896, 896, 4, 6), (192, 896, 4864, 7, 1)]:
        x, w = randn_bf16(g, M, K), (randn_bf16(g, N, K) / K ** 0.5).to(BF)
        got = a8.gemm_small(x.to(dev), w.to(dev), splits=sp, ws=ws, mblocks=mb)
        torch.cuda.synchronize()
        _check(got, x, w)
    assert (ws[:4096] == 0).all()


def test_gemm_dispatch_graph(a8, dev):
    """A tuned GemmDispatch (one shape where gemm_small applies, one where it does not) captured in a graph:
    every replay equals the eager call bit for bit."""
    say("case: GemmDispatch tuned, graph replays")
    g = torch.Generator().manual_seed(5)
    w1, w2 = randn_bf16(g, 896, 896).to(dev), randn_bf16(g, 896, 4864).to(dev)
    mm = a8.GemmDispatch()
    mm.tune([w1, w2], [192, 300])
    x1, x2 = randn_bf16(g, 192, 896).to(dev), randn_bf16(g, 192, 4864).to(dev)
    x3 = randn_bf16(g, 300, 896).to(dev)          # M > 192: the library GEMM
    assert mm.small[(300, 896, 896)] is None
    eager = [mm(x1, w1), mm(x2, w2), mm(x3, w1)]
    outs = [None, None, None]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mm(x1, w1)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [mm(x1, w1), mm(x2, w2), mm(x3, w1)]
    for _ in range(3):
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e)
    say(f"  choices {mm.small}")


def test_gemm_dispatch_tuning_cache(a8, dev, tmp_path):
    """tune(..., cache_path) writes its choices (small M, the gated launch, the prefill-sized record) into a JSON
    file keyed by GPU; a second dispatcher tuned from that file times nothing and makes the same choices, and
    an entry missing from the file is timed and merged in."""
    say("case: GemmDispatch tuning cache round trip")
    import json
    g = torch.Generator().manual_seed(9)
    wq, w13 = randn_bf16(g, 1152, 896).to(dev), randn_bf16(g, 2 * 512, 896).to(dev)
    path = str(tmp_path / "gemm_tune.json")
    a = a8.GemmDispatch()
    a.tune([wq, w13], [192], gated=[w13], large_m=1024, cache_path=path)
    disk = json.load(open(path))
    key = a8.GemmDispatch.gpu_key(dev)
    assert set(disk) == {key}
    assert {"s192,1152,896", "s192,1024,896", "g192,1024,896", "l1152,896", "l1024,896"} <= set(disk[key])
    assert a.large[(1152, 896)]["choice"] == "library"

    b = a8.GemmDispatch()
    timed = []
    orig = b._time
    b._time = lambda *args, **kw: timed.append(1) or orig(*args, **kw)
    b.tune([wq, w13], [192], gated=[w13], large_m=1024, cache_path=path)
    assert not timed
    assert b.small == a.small and b.small_best == a.small_best and b.gated_best == a.gated_best
    assert b.large == a.large
    x = randn_bf16(g, 192, 896).to(dev)
    assert torch.equal(b(x, wq), a(x, wq))

    # a new token count is timed and merged; the earlier entries stay
    b.tune([wq], [64], large_m=1024, cache_path=path)
    assert timed
    disk = json.load(open(path))[key]
    assert "s64,1152,896" in disk and "s192,1152,896" in disk


@pytest.mark.parametrize("M,I,K,mblocks", [(192, 4864, 896, 1), (192, 4864, 896, 3), (37, 1000, 640, 1),
                                           (100, 24, 128, 2), (1, 8, 64, 1)])
def test_gemm_silu_small(a8, dev, M, I, K, mblocks):
    """The w13 product with SiLU-mul in its epilogue equals gemm_small then silu_mul bit for bit (the slow AR's
    4864-wide MLP; ragged I with a partial last tile; row blocks), and that pair matches the oracle's
    linear + silu_mul (oracle/layer_ref.py) within the GEMM's bar."""
    say(f"case: gemm_silu M={M} I={I} K={K} mblocks={mblocks}")
    from oracle import layer_ref
    g = torch.Generator().manual_seed(M + I + K)
    x, w13 = randn_bf16(g, M, K), (randn_bf16(g, 2 * I, K) / K ** 0.5).to(BF)
    xd, wd = x.to(dev), w13.to(dev)
    got = a8.gemm_silu_small(xd, wd, mblocks=mblocks)
    pair = a8.silu_mul(a8.gemm_small(xd, wd))
    torch.cuda.synchronize()
    assert torch.equal(got, pair)
    gu = a8.gemm_small(xd, wd).cpu()
    _check(gu, x, w13)
    want = layer_ref.silu_mul(gu)
    assert torch.equal(pair.cpu(), want) or (pair.cpu().float() - want.float()).abs().max().item() <= \
        2 ** -7 * want.float().abs().max().item()


def test_dispatch_gated_takes_the_fused_launch(a8, dev):
    """GemmDispatch.gated: the fused launch where the tuned w13 choice is gemm_small without k splits (forced
    here), silu_mul(product) otherwise; both equal silu_mul(dispatch(x, w13))."""
    say("case: GemmDispatch.gated")
    g = torch.Generator().manual_seed(3)
    x, w13 = randn_bf16(g, 192, 896).to(dev), (randn_bf16(g, 2 * 512, 896) / 30.0).to(BF).to(dev)
    mm = a8.GemmDispatch()
    mm.small[(192, 1024, 896)] = (1, 1)
    a = mm.gated(x, w13)
    b = a8.silu_mul(mm(x, w13))
    mm.small[(192, 1024, 896)] = None          # the library product, then silu_mul
    c = mm.gated(x, w13)
    d = a8.silu_mul(torch.matmul(x, w13.t()))
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(c, d)
