"""The streaming vocoder's channels-last convolutions on the GPU (conv_cl, snake_cat) against the oracle
(oracle/conv_ref.py, pinned to torch's conv1d / conv_transpose1d): the codec decoder's conv shapes (input
conv, the stride-s transposed convs as phases, residual units' dilated k=7 conv and 1x1 conv with the snake on
the load and the residual, the one-channel output conv), ragged sizes, and the decoder's call pattern
(snake_cat into the conv, the state refreshed from the concatenated input)."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
F16 = torch.float16


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def cref():
    from oracle import conv_ref
    return conv_ref


def _close(got, want):
    """fp16 results: within one fp16 ulp of the oracle (fp32 sums in another order), or 1e-3 of the output
    scale where a sum cancels."""
    g, w = got.cpu().float(), want.float()
    ulp = (w.abs() * 2 ** -10).clamp(min=2 ** -24)
    scale = w.abs().max().item()
    return bool((((g - w).abs() <= ulp * 1.01) | ((g - w).abs() <= 1e-3 * scale)).all())


@pytest.mark.parametrize("B,T,Cin,Cout,cw,taps,dil,ph,bias,res,snake", [
    (8, 4, 1024, 768, 768, 7, 1, 1, True, False, False),      # input conv
    (8, 4, 768, 384, 384, 2, 1, 8, True, False, False),       # stride-8 transposed conv as 8 phases
    (8, 64, 96, 96, 96, 7, 9, 1, True, False, False),         # residual unit's dilated conv (after snake_cat)
    (8, 64, 96, 96, 96, 1, 1, 1, True, True, True),           # residual unit's 1x1 conv, snake on load, + input
    (8, 128, 96, 1, 16, 7, 1, 1, True, False, False),         # one-channel output conv (padded weights)
    (3, 5, 8, 24, 32, 3, 2, 3, False, True, True),            # ragged: one k chunk, Cout 24, 15 rows
    (4, 8, 512, 30, 32, 7, 1, 1, True, True, True),           # split K with Cout 30 (no 4-channel vectors)
    (64, 1024, 192, 192, 192, 1, 1, 1, True, True, True),     # long pointwise convs (block 2's shape)
    (65, 1009, 96, 96, 96, 1, 1, 1, True, True, True),        #   (ragged last tile)
    (64, 1100, 96, 24, 32, 1, 1, 1, False, True, False),      #   (Cout 24, no bias, no snake)
    (64, 1030, 192, 70, 80, 1, 1, 1, True, False, True),      #   (Cout 70: element stores)
])
def test_conv_cl_shapes(a8, cref, dev, B, T, Cin, Cout, cw, taps, dil, ph, bias, res, snake):
    say(f"case: conv_cl B={B} T={T} Cin={Cin} Cout={Cout} taps={taps} dil={dil} ph={ph} bias={bias} res={res} "
        f"snake={snake}")
    g = torch.Generator().manual_seed(B + T + Cin + Cout + taps)
    Tin = T + (taps - 1) * dil
    x = torch.randn(B, Tin, Cin, generator=g).to(F16)
    w = (torch.randn(ph, taps, Cin, cw, generator=g) / (taps * Cin) ** 0.5).to(F16)
    bv = torch.randn(cw, generator=g).to(F16) if bias else None
    rv = torch.randn(B, T * ph, Cout, generator=g).to(F16) if res else None
    ab = None
    if snake:
        a = (torch.rand(Cin, generator=g) + 0.5)
        ab = (a, 1.0 / (a + 1e-9))
    want = cref.conv_cl(x, w, bv, T, taps, dil, ph, Cout, res=rv, snake_ab=ab)
    out = torch.full((B, T * ph, Cout), 7.0, dtype=F16, device=dev)
    nws = a8.conv_cl_ws_bytes(B, T, Cin, Cout, taps, ph)      # the split-K shapes get a caller workspace
    ws = torch.empty(nws, dtype=torch.uint8, device=dev) if nws > 0 else None
    a8.conv_cl(x.to(dev), w.to(dev), bv.to(dev) if bias else None, T, taps, dil, ph, out,
               res=rv.to(dev) if res else None, snake=(ab[0].to(dev), ab[1].to(dev)) if snake else None, ws=ws)
    torch.cuda.synchronize()
    assert _close(out, want)


@pytest.mark.parametrize("Cout,cw", [(30, 32), (1, 16), (96, 96)])
def test_conv_cl_into_offset_view(a8, cref, dev, Cout, cw):
    """out (and res) as time-offset views of a larger buffer, as the reference's conv_cl accepts: row 1
    onwards, so the view starts 2 * Cout bytes in (not 8-byte aligned for odd Cout / 2); the rows around it
    are left alone."""
    say(f"case: conv_cl into out[:, 1:] with Cout={Cout}")
    g = torch.Generator().manual_seed(40 + Cout)
    B, T, Cin, taps = 3, 9, 64, 3
    x = torch.randn(B, T + taps - 1, Cin, generator=g).to(F16)
    w = (torch.randn(1, taps, Cin, cw, generator=g) / (taps * Cin) ** 0.5).to(F16)
    bv = torch.randn(cw, generator=g).to(F16)
    rbuf = torch.randn(B, T + 1, Cout, generator=g).to(F16)
    want = cref.conv_cl(x, w, bv, T, taps, 1, 1, Cout, res=rbuf[:, 1:])
    buf = torch.full((B, T + 2, Cout), 7.0, dtype=F16, device=dev)
    rb_d = rbuf.to(dev)
    a8.conv_cl(x.to(dev), w.to(dev), bv.to(dev), T, taps, 1, 1, buf[:, 1:T + 1], res=rb_d[:, 1:])
    torch.cuda.synchronize()
    got = buf.cpu()
    assert _close(got[:, 1:T + 1], want)
    assert (got[:, 0] == 7.0).all() and (got[:, T + 1] == 7.0).all()


def test_snake_cat_and_decoder_call_pattern(a8, cref, dev):
    """_CLConv.__call__ (fast_engine.py:218-233) for a context conv, frame after frame: snake_cat(x, state) into
    the conv's input, conv_cl over it, the state refreshed from the input's last ctx rows; against the oracle
    doing the same."""
    say("case: snake_cat + conv_cl streaming over 5 chunks")
    g = torch.Generator().manual_seed(91)
    B, C, Cout, taps, dil = 4, 96, 96, 7, 3
    ctx = (taps - 1) * dil
    w = (torch.randn(1, taps, C, Cout, generator=g) / (taps * C) ** 0.5).to(F16)
    bias = torch.randn(Cout, generator=g).to(F16)
    a = torch.rand(C, generator=g) + 0.5
    ib = 1.0 / (a + 1e-9)
    st_d = torch.zeros(B, ctx, C, dtype=F16, device=dev)
    wd, bd, ad, ibd = w.to(dev), bias.to(dev), a.to(dev), ib.to(dev)
    for T in (1, 5, 32, 2, 64):
        x = torch.randn(B, T, C, generator=g).to(F16)
        st_h = st_d.cpu()                   # the oracle continues from the device's state (snake rows may differ
        xin = torch.empty(B, ctx + T, C, dtype=F16, device=dev)   # from the oracle's by one fp16 ulp)
        a8.snake_cat(x.to(dev), st_d, ad, ibd, xin)
        y = torch.empty(B, T, Cout, dtype=F16, device=dev)
        a8.conv_cl(xin, wd, bd, T, taps, dil, 1, y)
        st_d.copy_(xin[:, T:])
        xin_h = cref.snake_cat(x, st_h, a, ib)
        torch.cuda.synchronize()
        assert torch.equal(xin.cpu()[:, :ctx], st_h)                          # the state rows move verbatim
        assert _close(xin[:, ctx:], xin_h[:, ctx:])                           # the snake: <= 1 fp16 ulp
        assert _close(y, cref.conv_cl(xin.cpu(), w, bias, T, taps, dil, 1, Cout))
        assert _close(y, cref.conv_cl(xin_h, w, bias, T, taps, dil, 1, Cout))


def test_conv_cl_split_k_equals_one_pass(a8, dev):
    """The split-K path (short input, long K: the decoder's input conv) gives the same bits as the one-pass
    kernel the entry point runs without a workspace: both sum in fp32, the split sums its shares in a fixed
    order, so only the association differs -- checked to one fp16 ulp, and run-to-run identical."""
    say("case: conv_cl split-K vs one pass, B=8 T=4 Cin=1024 Cout=1536 taps=7")
    lib = a8.load_library()
    g = torch.Generator(device=dev).manual_seed(4)
    B, T, Cin, Cout, taps = 8, 4, 1024, 1536, 7
    x = torch.randn(B, T + taps - 1, Cin, generator=g, device=dev).to(F16)
    w = (torch.randn(1, taps, Cin, Cout, generator=g, device=dev) / (taps * Cin) ** 0.5).to(F16)
    bias = torch.randn(Cout, generator=g, device=dev).to(F16)
    nws = lib.a8_conv_cl_ws_bytes(B, T, Cin, Cout, taps, 1)
    assert nws > 0
    ws = torch.empty(nws, dtype=torch.uint8, device=dev)
    outs = []
    for use_ws in (True, True, False):
        y = torch.empty(B, T, Cout, dtype=F16, device=dev)
        st = lib.a8_conv_cl(x.data_ptr(), x.stride(0), x.stride(1), w.data_ptr(), w.stride(0), w.stride(1),
                            w.stride(2), Cout, bias.data_ptr(), None, 0, 0, y.data_ptr(), y.stride(0), y.stride(1),
                            None, None, B, x.shape[1], T, Cin, Cout, taps, 1, 1, ws.data_ptr() if use_ws else None,
                            nws if use_ws else 0, torch.cuda.current_stream().cuda_stream)
        assert st == 0
        outs.append(y)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    d = (outs[0].float() - outs[2].float()).abs()
    assert (d <= outs[2].float().abs() * 2 ** -10 + 1e-3).all()


@pytest.mark.parametrize("B,T,C,dil", [(8, 64, 96, 9), (8, 64, 192, 3), (64, 1024, 192, 1), (65, 1009, 96, 3),
                                       (3, 5, 96, 9), (2, 130, 192, 9), (64, 256, 384, 3), (5, 70, 384, 9)])
def test_ru_cl_against_oracle(a8, cref, dev, B, T, C, dil):
    """A whole residual unit in one launch (ru_cl) against the oracle's ru_fused: snake_cat of the state and
    the raw input, then the fused k=7 conv, second snake, 1x1 conv, bias and residual; long inputs (block 2 /
    3 row counts), a ragged last tile, T shorter than the context, every dilation of the decoder."""
    say(f"case: ru_cl B={B} T={T} C={C} dil={dil}")
    g = torch.Generator().manual_seed(B * 7 + C + dil)
    taps = 7
    ctx = (taps - 1) * dil
    x = torch.randn(B, T, C, generator=g).half()
    st = torch.randn(B, ctx, C, generator=g).half()
    a1, a2 = torch.rand(C, generator=g) + 0.5, torch.rand(C, generator=g) + 0.5
    ib1, ib2 = 1.0 / (a1 + 1e-9), 1.0 / (a2 + 1e-9)
    w1 = (torch.randn(taps, C, C, generator=g) / (taps * C) ** 0.5).half()
    w2 = (torch.randn(C, C, generator=g) / C ** 0.5).half()
    b1, b2 = (0.1 * torch.randn(C, generator=g)).half(), (0.1 * torch.randn(C, generator=g)).half()
    want = cref.ru_fused(x, st, a1, ib1, w1, b1, a2, ib2, w2, b2, taps, dil)
    xd = x.to(dev)
    xin = torch.empty(B, ctx + T, C, dtype=F16, device=dev)
    a8.snake_cat(xd, st.to(dev), a1.to(dev), ib1.to(dev), xin)
    out = torch.full((B, T, C), 9.0, dtype=F16, device=dev)
    a8.ru_cl(xin, w1.to(dev), b1.to(dev), a2.to(dev), ib2.to(dev), w2.to(dev), b2.to(dev), xd, out, T, taps, dil)
    torch.cuda.synchronize()
    assert torch.isfinite(out.cpu().float()).all()
    assert _close(out, want)


def test_ru_cl_refuses_other_widths(a8, dev):
    """Widths whose row does not fit one tile are refused (the caller takes the two convs)."""
    C = 768
    xin = torch.zeros(1, 10, C, dtype=F16, device=dev)
    w1, w2 = torch.zeros(7, C, C, dtype=F16, device=dev), torch.zeros(C, C, dtype=F16, device=dev)
    v16, v32 = torch.zeros(C, dtype=F16, device=dev), torch.zeros(C, device=dev)
    with pytest.raises(RuntimeError, match="ru_cl"):
        a8.ru_cl(xin, w1, v16, v32, v32, w2, v16, xin, torch.empty(1, 4, C, dtype=F16, device=dev), 4, 7, 1)


@pytest.mark.parametrize("B,T,C,taps", [(4, 2048, 96, 7), (3, 300, 96, 7), (2, 7, 32, 7), (5, 513, 128, 3),
                                      (3, 200, 40, 8), (2, 129, 8, 1)])
def test_conv_out_tanh_against_the_call_it_replaces(a8, cref, dev, B, T, C, taps):
    """conv_out_tanh (the decoder's last conv, one launch) against what it replaces, frame after frame: snake_cat,
    conv_cl into one channel (padded weights), the state copy and tanh -- on the device (the state bit for bit,
    the fp16 conv output within one ulp: another summation order; tanh of it within 2e-3) and the oracle."""
    say(f"case: conv_out_tanh B={B} T={T} C={C} taps={taps}")
    g = torch.Generator().manual_seed(B * T + C)
    ctx = taps - 1
    w = (torch.randn(taps, C, generator=g) / (taps * C) ** 0.5).to(F16)
    W = torch.zeros(1, taps, C, 16, dtype=F16)
    W[0, :, :, 0] = w
    bias = torch.randn(1, generator=g).to(F16)
    a = torch.rand(C, generator=g) + 0.5
    ib = 1.0 / (a + 1e-9)
    wd, Wd, bd, ad, ibd = w.to(dev), W.to(dev), bias.to(dev), a.to(dev), ib.to(dev)
    st1 = torch.zeros(B, ctx, C, dtype=F16, device=dev)
    st2 = st1.clone()
    for rep in range(3):
        x = (torch.randn(B, T, C, generator=g) * 2).to(F16).to(dev)
        st_h = st2.cpu()
        y = torch.empty(B, T, dtype=torch.float32, device=dev)
        a8.conv_out_tanh(x, st1, ad, ibd, wd, bd, y)
        xin = torch.empty(B, ctx + T, C, dtype=F16, device=dev)
        a8.snake_cat(x, st2, ad, ibd, xin)
        y16 = torch.empty(B, T, 1, dtype=F16, device=dev)
        a8.conv_cl(xin, Wd, bd, T, taps, 1, 1, y16)
        st2.copy_(xin[:, T:])
        torch.cuda.synchronize()
        assert torch.equal(st1, st2), rep                                      # the new state, bit for bit
        want16 = cref.conv_cl(xin.cpu(), W, bias, T, taps, 1, 1, 1)[..., 0]    # the oracle on the same input
        assert _close(torch.atanh(y.cpu().clamp(-0.9999, 0.9999)).to(F16).unsqueeze(-1), y16.cpu()) or \
            (y.cpu() - torch.tanh(y16.cpu()[..., 0].float())).abs().max().item() <= 2e-3
        assert (y.cpu() - torch.tanh(want16.float())).abs().max().item() <= 2e-3, rep
        xin_h = cref.snake_cat(x.cpu(), st_h, a, ib)
        want_h = torch.tanh(cref.conv_cl(xin_h, W, bias, T, taps, 1, 1, 1)[..., 0].float())
        assert (y.cpu() - want_h).abs().max().item() <= 2e-3, rep


def test_decoder_fused_output_conv(dev):
    """The decoder with its last conv fused (the default) against the same decoder with snake_cat + conv_cl +
    state copy + tanh: waveforms within 2e-3, every state bit for bit, over several frames."""
    import importlib
    voc = importlib.import_module("audio8-turbo-engine_amd.vocoder")
    say("case: decoder, fused output conv vs the four-step call")
    wd = voc.decoder_weights(dev=dev, seed=31)
    d1, d2 = voc.CLDecoder(wd, 4, dev), voc.CLDecoder(wd, 4, dev)
    d2.fused_out = False
    assert d1.fused_out
    g = torch.Generator(device=dev).manual_seed(32)
    for rep in range(3):
        x = torch.randn(4, 4, 1024, generator=g, device=dev).to(F16)
        y1, y2 = d1(x, 4), d2(x, 4)
        torch.cuda.synchronize()
        assert (y1 - y2).abs().max().item() <= 2e-3, rep
        for s1, s2 in zip(d1.states, d2.states):
            assert torch.equal(s1, s2), rep


@pytest.mark.parametrize("snake", [True, False])
def test_snake_cat_refresh_equals_copy(a8, dev, snake):
    """snake_cat(..., refresh=True) against snake_cat then the state copy the reference makes after the conv
    (fast_engine.py:232): the concatenated rows and the next state bit for bit, frame after frame, including
    frames exactly as long as the context."""
    say(f"case: snake_cat refresh, snake {snake}")
    g = torch.Generator().manual_seed(93)
    B, C, ctx = 5, 96, 18
    a = (torch.rand(C, generator=g) + 0.5).to(dev) if snake else None
    ib = (1.0 / (a + 1e-9)) if snake else None
    s1 = torch.randn(B, ctx, C, generator=g).to(F16).to(dev)
    s2 = s1.clone()
    for T in (18, 64, 19, 1024):
        x = torch.randn(B, T, C, generator=g).to(F16).to(dev)
        y1 = torch.empty(B, ctx + T, C, dtype=F16, device=dev)
        y2 = torch.empty_like(y1)
        a8.snake_cat(x, s1, a, ib, y1, refresh=True)
        a8.snake_cat(x, s2, a, ib, y2)
        s2.copy_(y2[:, T:])
        torch.cuda.synchronize()
        assert torch.equal(y1, y2), T
        assert torch.equal(s1, s2), T
    with pytest.raises(Exception):  # shorter than the context: refused (the caller copies instead)
        a8.snake_cat(torch.zeros(B, 4, C, dtype=F16, device=dev), s1, a, ib,
                     torch.empty(B, ctx + 4, C, dtype=F16, device=dev), refresh=True)
