"""The norm-fused projections (gemm_small_norm) and the slow stack that uses them (SlowStack.fuse_norm), on the
GPU through the C ABI: the residual add bit for bit against gemm_small's rounded product plus torch's bf16 add,
its per-row sums of squares against torch; the RMSNorm consumer (the norm weight folded into the weight, the
norm's 1 / rms on the fp32 products) against a float64 evaluation, plain and with the gated SiLU epilogue; the
fused 24-layer-shaped step against the oracle's _Stack.forward restatement, and its graph replays against the
eager step."""
from __future__ import annotations

import pytest
import torch

from conftest import randn_bf16

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def lref():
    from oracle import layer_ref
    return layer_ref


def _ulps(a, b):
    return (a.view(torch.int16).int() - b.view(torch.int16).int()).abs()


@pytest.mark.parametrize("M,N,K,splits,mblocks", [(192, 896, 896, 1, 6), (192, 896, 4864, 4, 3), (64, 896, 896, 1, 1),
                                                  (192, 896, 4864, 1, 1), (40, 256, 512, 2, 1)])
def test_residual_add_and_sums_of_squares(a8, dev, M, N, K, splits, mblocks):
    say(f"case: gemm_small_norm res_add M={M} N={N} K={K} splits={splits} mblocks={mblocks}")
    g = torch.Generator().manual_seed(M + N + K)
    x = randn_bf16(g, M, K).to(dev)
    w = (randn_bf16(g, N, K) * (K ** -0.5)).to(BF).to(dev)
    res0 = randn_bf16(g, M, N).to(dev)
    ws = torch.zeros(a8.gemm_ws_bytes(M, N, splits), dtype=torch.uint8, device=dev) if splits > 1 else None
    a = a8.gemm_small(x, w, splits=splits, ws=ws, mblocks=mblocks)
    want = (a.float() + res0.float()).to(BF)
    res = res0.clone()
    ss = torch.full((M, N // 32), -1.0, dtype=torch.float32, device=dev)
    for rep in range(2):  # the workspace counters are left at zero: a second call is the same
        res.copy_(res0)
        a8.gemm_small_norm(x, w, res, splits=splits, mblocks=mblocks, ws=ws, res_add=True, ss_out=ss)
        torch.cuda.synchronize()
        assert torch.equal(res, want), (rep, _ulps(res, want).max().item())
    ss_want = (want.float() ** 2).view(M, N // 32, 32).sum(-1)
    assert torch.allclose(ss, ss_want, rtol=1e-5, atol=1e-5), (ss - ss_want).abs().max().item()


@pytest.mark.parametrize("M,N,K,splits,mblocks,gated", [(192, 1152, 896, 1, 6, False), (192, 9728, 896, 1, 1, True),
                                                        (64, 1152, 896, 3, 1, False), (33, 256, 512, 1, 1, True)])
def test_norm_consumer_against_float64(a8, lref, dev, M, N, K, splits, mblocks, gated):
    """out = bf16(h @ fold_norm(w, ln)^T * rsqrt(mean(h^2) + eps)), the statistic from 32-column sums of
    squares as a producer leaves them; within 2 bf16 ulps of float64 (the gated one: of silu_mul of the two
    float64 halves rounded to bf16, within one more ulp where the halves' roundings differ)."""
    say(f"case: gemm_small_norm consumer M={M} N={N} K={K} splits={splits} mblocks={mblocks} gated={gated}")
    g = torch.Generator().manual_seed(7 * M + N)
    h = (randn_bf16(g, M, K) * 3).to(BF)
    w = (randn_bf16(g, N, K) * (K ** -0.5)).to(BF)
    ln = (1 + 0.05 * torch.randn(K, generator=g)).to(BF)
    eps = 1e-6
    wf = a8.fold_norm(w, ln)
    ss = (h.float() ** 2).view(M, K // 32, 32).sum(-1).contiguous()
    inv = torch.rsqrt((h.double() ** 2).mean(-1, keepdim=True) + eps)
    prod = (h.double() @ wf.double().t()) * inv
    ws = torch.zeros(a8.gemm_ws_bytes(M, N, splits), dtype=torch.uint8, device=dev) if splits > 1 else None
    out = torch.empty(M, N // 2 if gated else N, dtype=BF, device=dev)
    a8.gemm_small_norm(h.to(dev), wf.to(dev), out, splits=splits, mblocks=mblocks, ws=ws, gated=gated,
                       ss_in=ss.to(dev), eps=eps)
    torch.cuda.synchronize()
    got = out.cpu()
    # the bar of gemm_small's own tests: 2 bf16 ulps of the value plus 1e-3 of the largest (fp32 sums cancel
    # on near-zero outputs); gated: of silu_mul over the float64 halves rounded to bf16, one ulp more
    want = lref.silu_mul(prod.to(BF)).double() if gated else prod
    bar = 3 if gated else 2
    err = (got.double() - want).abs()
    tol = bar * 2.0 ** -8 * want.abs() + 1e-3 * want.abs().max()
    u = _ulps(got, want.to(BF))
    say(f"  max ulps {u.max().item()}, exact {(u == 0).float().mean().item():.4f}, worst err / tol "
        f"{(err / tol).max().item():.3f}")
    assert (err <= tol).all()


@pytest.mark.parametrize("M,N,K,splits,mblocks", [(192, 1152, 896, 1, 6), (192, 9728, 896, 1, 1),
                                                  (64, 1152, 896, 3, 1), (33, 256, 512, 1, 1)])
def test_folded_norm_against_reference_sequence(a8, lref, dev, M, N, K, splits, mblocks):
    """The folded-norm product (norm weight folded into the weight, 1 / rms on the fp32 products) against the
    reference's own sequence as the oracle restates it: rmsnorm (two bf16 roundings) then the bf16 product
    (fast_kernels.py:30-46, fast_engine.py:90). Two bars:
      * absolute, every element: with u = 2^-8 (bf16) and t_k = h_k r g_k w_nk, the reference rounds each
        term's factors twice and the fused path once, so |got - ref| <= 3u sum|t_k| + 2 gamma_K sum|t_k|
        + u (|got| + |ref|) (gamma_K = K 2^-24 for the fp32 sums; the last term: each output's own rounding);
      * statistical: the roundings are independent, so the RMS difference stays within 2u of the RMS output;
        a dropped or misplaced factor (norm weight, 1 / rms, eps) moves it by percents."""
    say(f"case: folded norm vs rmsnorm -> product M={M} N={N} K={K} splits={splits} mblocks={mblocks}")
    g = torch.Generator().manual_seed(3 * M + N + K)
    h = (randn_bf16(g, M, K) * 3).to(BF)
    w = (randn_bf16(g, N, K) * (K ** -0.5)).to(BF)
    ln = (1 + 0.05 * torch.randn(K, generator=g)).to(BF)
    eps = 1e-6
    y, _ = lref.rmsnorm(h, ln, eps)
    ref_out = lref.linear(y, w).double()
    ss = (h.float() ** 2).view(M, K // 32, 32).sum(-1).contiguous()
    ws = torch.zeros(a8.gemm_ws_bytes(M, N, splits), dtype=torch.uint8, device=dev) if splits > 1 else None
    out = torch.empty(M, N, dtype=BF, device=dev)
    a8.gemm_small_norm(h.to(dev), a8.fold_norm(w, ln).to(dev), out, splits=splits, mblocks=mblocks, ws=ws,
                       ss_in=ss.to(dev), eps=eps)
    torch.cuda.synchronize()
    got = out.cpu().double()
    hd = h.double()
    r = torch.rsqrt((hd ** 2).mean(-1, keepdim=True) + eps)
    tabs = (hd.abs() * r) @ (w.double().abs() * ln.double().abs()).t()   # sum_k |t_k|
    u, gam = 2.0 ** -8, K * 2.0 ** -24
    bound = (3 * u + 2 * gam) * tabs + u * (got.abs() + ref_out.abs())
    diff = (got - ref_out).abs()
    rms_d, rms_y = diff.pow(2).mean().sqrt().item(), ref_out.pow(2).mean().sqrt().item()
    say(f"  max |diff| {diff.max().item():.3e}, worst diff / bound {(diff / bound).max().item():.3f}, "
        f"RMS diff / RMS out {rms_d / rms_y:.2e} (bar {2 * u:.2e})")
    assert (diff <= bound).all()
    assert rms_d <= 2 * u * rms_y


def test_slow_stack_fused_norm(a8, ref, lref, dev):
    """The decode tick with fuse_norm (every projection on gemm_small, the norms inside them) at the slow AR's
    widths and 192 rows against the oracle, with the same bar as the unfused stack, and its graph replays
    against the eager step bit for bit."""
    import importlib
    tl = importlib.import_module("test_gpu_layer")
    say("case: slow stack, norm-fused projections, 192 rows")
    n_layers, hidden, inter, b, S = 3, 896, 4864, 192, 256
    st, layers, norm = tl._stack(a8, dev, n_layers, hidden, inter, b, S, seed=23)
    mm = a8.GemmDispatch()
    mm.tune([L[k] for L in layers for k in ("wqkv", "wo", "w13", "w2")], [b], gated=[L["w13"] for L in layers])
    st.mm = mm
    st.fuse_norm = True
    g = torch.Generator().manual_seed(24)
    x = randn_bf16(g, b, hidden)
    lens = torch.randint(1, S + 1, (b,), generator=g).int()
    pos, slot = lens - 1, torch.arange(b, dtype=torch.int32)
    kc0 = [t.clone() for t in st.kc]
    vc0 = [t.clone() for t in st.vc]
    kc = [t.cpu() for t in st.kc]
    vc = [t.cpu() for t in st.vc]
    want = lref.slow_stack(x.clone(), pos, slot, lens, tl._cpu(layers), norm.cpu(), tl.NQ, tl.NKV, tl.HD, 1e-6,
                           st.attn.cos.cpu(), st.attn.sin.cpu(), kc, vc, rowmap=False)
    xd, posd, slotd, lensd = x.to(dev), pos.to(dev), slot.to(dev), lens.to(dev)
    # the same step unfused (the reference's rmsnorm -> product sequence, bit for bit but for GEMM summation
    # order): its distance to the oracle is the rounding noise the fused step is held to
    st.fuse_norm = False
    ref_step = st.forward(xd.clone(), posd, slotd, lensd, rowmap=False, fuse=True).clone()
    for i in range(n_layers):
        st.kc[i].copy_(kc0[i])
        st.vc[i].copy_(vc0[i])
    st.fuse_norm = True
    got = st.forward(xd.clone(), posd, slotd, lensd, rowmap=False, fuse=True).clone()
    torch.cuda.synchronize()
    emax, emean, vmax = tl._close(got, want)
    umax, umean, _ = tl._close(ref_step, want)
    say(f"  fused: max-abs {emax:.3e} mean-abs {emean:.3e}; unfused: max-abs {umax:.3e} mean-abs {umean:.3e} "
        f"(max |h| {vmax:.2f}); choices {mm.small}")
    # the unfused stack's bar for the largest error; the mean error within 2x the unfused step's: the fused step
    # rounds at other points (the folded weight instead of each norm's two bf16 outputs), perturbations of the
    # same size that add to the unfused step's GEMM-order noise (about sqrt(2) x expected)
    assert emax <= 0.02 * vmax and emean <= max(5e-3, 2.0 * umean)
    for i in range(n_layers):
        dk = (st.kc[i].cpu().float() - kc[i].float()).abs().max().item()
        assert dk <= 0.05, dk
    xbuf = torch.empty_like(xd)

    def step():
        return st.forward(xbuf, posd, slotd, lensd, rowmap=False, fuse=True)

    for i in range(n_layers):
        st.kc[i].copy_(kc0[i])
        st.vc[i].copy_(vc0[i])
    xbuf.copy_(xd)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        yg = step()
    for rep in range(3):
        for i in range(n_layers):
            st.kc[i].copy_(kc0[i])
            st.vc[i].copy_(vc0[i])
        xbuf.copy_(xd)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, got), f"replay {rep} differs from the eager step"


def test_prefetch_workgroups_change_nothing(a8, dev):
    """gemm_small_norm with prefetch workgroups in its grid (the next product's weights read beside it) gives the
    same residual stream and sums of squares as without, bit for bit, at one and four k splits; and a prefetch
    that covers a ragged byte count (not a multiple of the grid's stride) reads within its tensor."""
    say("case: gemm_small_norm with prefetch workgroups vs without")
    g = torch.Generator().manual_seed(91)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    nxt = randn_bf16(g, 9728 * 896 + 40, 1).view(-1).to(dev)   # 17.4 MB + 80 bytes
    for M, N, K, splits, mblocks in ((192, 896, 896, 1, 6), (192, 896, 4864, 4, 3)):
        x = randn_bf16(g, M, K).to(dev)
        w = (randn_bf16(g, N, K) * (K ** -0.5)).to(BF).to(dev)
        res0 = randn_bf16(g, M, N).to(dev)
        ws = torch.zeros(a8.gemm_ws_bytes(M, N, splits), dtype=torch.uint8, device=dev) if splits > 1 else None
        outs = []
        for pf in (None, nxt):
            res = res0.clone()
            ss = torch.zeros(M, N // 32, dtype=torch.float32, device=dev)
            a8.gemm_small_norm(x, w, res, splits=splits, mblocks=mblocks, ws=ws, res_add=True, ss_out=ss,
                               prefetch=pf, pf_sink=sink)
            torch.cuda.synchronize()
            outs.append((res, ss))
        assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1]), (M, N, K)


def test_slow_stack_prefetch_is_the_same_step(a8, dev):
    """The norm-fused slow-AR step with the w13 prefetch (the default) and the K-cache prefetch (opt-in) against
    the same step without either: the final hidden state and the caches bit for bit."""
    say("case: slow stack fused step, w13 + K prefetch on / off")
    from importlib import import_module
    ss_mod = import_module(a8.__name__ + ".slow_stack")
    layers, norm = ss_mod.random_weights(2, 896, 14, 2, 64, 1024, dev, seed=13)
    outs = []
    for pf in (True, False):
        st = a8.SlowStack(layers, norm, 14, 2, 64, 1e-6, 10000.0, max_rows=64, cache_rows=17, cache_len=256,
                          max_pos=256, dev=dev)
        mm = a8.GemmDispatch()
        mm.tune([L[k] for L in layers for k in ("wqkv", "wo", "w13", "w2")], [16], gated=[L["w13"] for L in layers])
        st.mm, st.fuse_norm, st.prefetch_w13 = mm, True, pf
        st.prefetch_kv_bytes = (1 << 20) if pf else 0
        gen = torch.Generator(device=dev).manual_seed(14)
        st.kc_all.normal_(generator=gen)
        st.vc_all.normal_(generator=gen)
        x = torch.randn(16, 896, generator=gen, device=dev).to(BF)
        lens = torch.full((16,), 200, dtype=torch.int32, device=dev)
        h = st.forward(x, lens - 1, torch.arange(16, dtype=torch.int32, device=dev), lens, rowmap=False, fuse=True)
        torch.cuda.synchronize()
        outs.append((h.clone(), st.kc_all.clone(), st.vc_all.clone()))
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)
