"""The streaming channels-last decoder (vocoder.CLDecoder on conv_cl / snake_cat) against the oracle's
whole-utterance decode (oracle/conv_ref.decoder: torch conv1d / conv_transpose1d, float64): streaming frame
chunks from zero state reproduce the whole-utterance decode (fast_engine.py:24-25), and rows are independent:
resetting one row's state restarts that row alone (work/voc_check.py's row independence)."""
from __future__ import annotations

import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def _small(dev):
    voc = importlib.import_module("audio8-turbo-engine_amd.vocoder")
    return voc, voc.decoder_weights(cin=64, ch=128, rates=(4, 2), k=7, dils=(1, 3, 9), dev="cpu", seed=3)


def test_streaming_decoder_matches_whole_utterance(dev):
    from oracle import conv_ref
    say("case: CLDecoder 64->128 ch, rates 4,2, chunks 1,2,3,1 x 3 rows")
    voc, wts = _small(dev)
    wd = {"conv_in": tuple(t.to(dev) for t in wts["conv_in"]),
          "blocks": [(a.to(dev), w.to(dev), b.to(dev), s, [tuple(t.to(dev) if torch.is_tensor(t) else t for t in u)
                                                          for u in us]) for a, w, b, s, us in wts["blocks"]],
          "final": tuple(t.to(dev) for t in wts["final"])}
    dec = voc.CLDecoder(wd, 4, dev)
    g = torch.Generator().manual_seed(8)
    B, chunks = 3, (1, 2, 3, 1)
    x = torch.randn(B, sum(chunks), 64, generator=g)
    outs, t0 = [], 0
    for T in chunks:
        outs.append(dec(x[:, t0:t0 + T].to(dev), B))
        t0 += T
    got = torch.cat(outs, 1).cpu().double()
    want = conv_ref.decoder(wts, x)
    torch.cuda.synchronize()
    assert got.shape == want.shape == (B, sum(chunks) * 8)
    err = (got - want).abs()
    say(f"max err {err.max().item():.2e} mean {err.mean().item():.2e} scale {want.abs().max().item():.3f}")
    assert err.max().item() < 2e-2 and err.mean().item() < 2e-3


def test_streaming_decoder_with_fused_units(dev):
    """A decoder whose blocks are 192 and 96 channels wide, so every residual unit runs fused (ru_cl): streaming
    chunks (shorter and longer than the units' contexts) reproduce the oracle's whole-utterance decode, and the
    two-conv decoder (the default, fused_ru=()) agrees with it as closely."""
    from oracle import conv_ref
    say("case: CLDecoder 64->384 ch, rates 2,2 (blocks of 192 / 96 channels: fused units), chunks 1,5,2 x 2 rows")
    voc = importlib.import_module("audio8-turbo-engine_amd.vocoder")
    wts = voc.decoder_weights(cin=64, ch=384, rates=(2, 2), k=7, dils=(1, 3, 9), dev="cpu", seed=5)
    wd = {"conv_in": tuple(t.to(dev) for t in wts["conv_in"]),
          "blocks": [(a.to(dev), w.to(dev), b.to(dev), s, [tuple(t.to(dev) if torch.is_tensor(t) else t for t in u)
                                                          for u in us]) for a, w, b, s, us in wts["blocks"]],
          "final": tuple(t.to(dev) for t in wts["final"])}
    dec, dec2 = voc.CLDecoder(wd, 2, dev, fused_ru=voc.FusedRU.DEFAULT_WIDTHS), voc.CLDecoder(wd, 2, dev)
    assert all(fu is not None for _, us in dec.blocks for _, _, fu in us)
    assert all(fu is None for _, us in dec2.blocks for _, _, fu in us)
    g = torch.Generator().manual_seed(10)
    B, chunks = 2, (1, 5, 2)
    x = torch.randn(B, sum(chunks), 64, generator=g)
    outs, outs2, t0 = [], [], 0
    for T in chunks:
        outs.append(dec(x[:, t0:t0 + T].to(dev), B))
        outs2.append(dec2(x[:, t0:t0 + T].to(dev), B))
        t0 += T
    got, got2 = torch.cat(outs, 1).cpu().double(), torch.cat(outs2, 1).cpu().double()
    want = conv_ref.decoder(wts, x)
    torch.cuda.synchronize()
    for name, y in (("fused", got), ("two-conv", got2)):
        err = (y - want).abs()
        say(f"{name}: max err {err.max().item():.2e} mean {err.mean().item():.2e}")
        assert err.max().item() < 2e-2 and err.mean().item() < 2e-3


def test_rows_are_independent(dev):
    say("case: CLDecoder row reset, 3 rows")
    voc, wts = _small(dev)
    wd = {"conv_in": tuple(t.to(dev) for t in wts["conv_in"]),
          "blocks": [(a.to(dev), w.to(dev), b.to(dev), s, [tuple(t.to(dev) if torch.is_tensor(t) else t for t in u)
                                                          for u in us]) for a, w, b, s, us in wts["blocks"]],
          "final": tuple(t.to(dev) for t in wts["final"])}
    g = torch.Generator().manual_seed(9)
    x1, x2 = torch.randn(3, 3, 64, generator=g).to(dev), torch.randn(3, 2, 64, generator=g).to(dev)
    dec = voc.CLDecoder(wd, 3, dev)
    dec(x1, 3)
    dec.reset_rows(torch.tensor([1], device=dev))
    y = dec(x2, 3)
    fresh = voc.CLDecoder(wd, 3, dev)(x2, 3)                  # every row from zero state
    cont = voc.CLDecoder(wd, 3, dev)
    cont(x1, 3)
    yc = cont(x2, 3)                                            # every row continuing
    torch.cuda.synchronize()
    assert torch.equal(y[1], fresh[1])
    assert torch.equal(y[0], yc[0]) and torch.equal(y[2], yc[2])
    assert not torch.equal(y[0], fresh[0])


def test_decoder_graph_replay_equals_eager(dev):
    """The decoder captured once as a graph (its split-K workspaces and activations from the graph's pool) and
    replayed frame after frame, with the program's own eager work between replays, gives the same bits as
    the eager decoder fed the same frames (fast_engine.py:744-768 captures the vocoder step in the tick)."""
    say("case: CLDecoder graph capture (256 channels: the input conv splits K), 4 replays vs eager")
    voc = importlib.import_module("audio8-turbo-engine_amd.vocoder")
    wts = voc.decoder_weights(cin=256, ch=256, rates=(2, 2), k=7, dils=(1, 3, 9), dev="cpu", seed=4)
    lib = importlib.import_module("audio8-turbo-engine_amd").load_library()
    assert lib.a8_conv_cl_ws_bytes(3, 2, 256, 256, 7, 1) > 0          # the input conv takes the split-K path
    wd = {"conv_in": tuple(t.to(dev) for t in wts["conv_in"]),
          "blocks": [(a.to(dev), w.to(dev), b.to(dev), s, [tuple(t.to(dev) if torch.is_tensor(t) else t for t in u)
                                                          for u in us]) for a, w, b, s, us in wts["blocks"]],
          "final": tuple(t.to(dev) for t in wts["final"])}
    B = 3
    dec_g, dec_e = voc.CLDecoder(wd, B, dev, frame=2), voc.CLDecoder(wd, B, dev, frame=2)
    assert dec_g.dec_in.ws is not None                                  # owned once, sized for the frame
    xs = torch.zeros(B, 2, 256, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        dec_g(xs, B)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        yg = dec_g(xs, B)
    rows = torch.arange(B, device=dev)
    dec_g.reset_rows(rows)
    gen = torch.Generator(device=dev).manual_seed(12)
    for f in range(4):
        x = torch.randn(B, 2, 256, generator=gen, device=dev)
        xs.copy_(x)
        graph.replay()
        ye = dec_e(x, B)
        torch.cuda.synchronize()
        assert torch.equal(yg, ye), f"frame {f}"
