"""The streaming codec decoder's convolution stack (reference serve/fast_engine.py:178-310: _CLConv, _CLDecoder)
on this package's conv kernels: channels-last fp16, one frame of work per frame, per-row causal state.

CLConv packs one causal Conv1d [Cout, Cin, K] (stride 1, dilation d) or one causal ConvTranspose1d
[Cin, Cout, 2s] (stride s, right crop s) into the weight layout conv_cl reads, [phases, taps, Cin, Cout_pad]
with Cout_pad = max(16, Cout) (fast_engine.py:183-206):
    Conv1d:           one phase, taps j = 0..K-1 at input rows t + j*d, ctx = (K-1)*d rows of state;
    ConvTranspose1d:  s phases, two taps: tap 0 reads the previous input frame with w[:, :, p + s], tap 1 the
                      current one with w[:, :, p]; ctx = 1 row of state.
Its call (fast_engine.py:218-233): without state the snake runs on the conv's loads; with state, snake_cat
builds [state, snake(x)] and conv_cl reads it, and the state keeps the last ctx activated rows.

CLDecoder (fast_engine.py:276-310): conv_in, then per block [snake + transposed conv, 3 residual units
(snake, dilated conv k, snake, 1x1 conv, + input)], snake + conv_out (one channel), tanh. The reference's
fused residual unit (_FusedRU, on for the widths TTS_VOC_FUSED_RU names) is FusedRU here, on ru_cl, and
`fused_ru` names its widths (ru_cl takes 96, 192 and 384). The default, (), keeps every unit as the two convs:
the reference's default (TTS_VOC_FUSED_RU unset), bit for bit its rounding sequence. FusedRU.DEFAULT_WIDTHS (96
and 192, where the fused unit measured faster; the benchmark's frame uses it) opts in. The fused unit keeps the
first conv's output in fp32 where the two convs round it to fp16, as the reference's fused unit does, so it
matches the two-conv decoder within fp16 rounding, not bit for bit.

The checkpoint's decoder (its modeling file and weights) is absent offline: `decoder_weights` draws a synthetic
decoder of a stated shape (default: a DAC-style 44.1 kHz decoder, 1024 -> 1536 channels, strides 8, 8, 4, 2,
kernel 7, dilations 1, 3, 9), with the reference's tensor layouts."""
from __future__ import annotations

import torch

from .fast_kernels import conv_cl, conv_cl_ws_bytes, conv_out_tanh, ru_cl, snake_cat

F16 = torch.float16


def pack_conv(w, trans=False, stride=1):
    """(W [ph, taps, Cin, Cout_pad] fp16, taps, ph) from a Conv1d weight [Cout, Cin, K] or a ConvTranspose1d
    weight [Cin, Cout, 2*stride] (fast_engine.py:186-206). Cout_pad = max(16, Cout) as in the reference,
    rounded up to a multiple of 8 (conv_cl reads weight rows 16 bytes at a time)."""
    w = w.detach().float()
    if trans:
        Cin, Cout, K = w.shape
        if K != 2 * stride:
            raise ValueError(f"transposed conv kernel {K} must be twice its stride {stride}")
        W = torch.stack([torch.stack([w[:, :, p + stride], w[:, :, p]]) for p in range(stride)])
        taps, ph = 2, stride
    else:
        Cout, Cin, K = w.shape
        W = w.permute(2, 1, 0).unsqueeze(0)
        taps, ph = K, 1
    Wp = torch.zeros(*W.shape[:-1], max(16, -(-Cout // 8) * 8), device=w.device)
    Wp[..., :Cout] = W
    return Wp.to(F16).contiguous(), taps, ph


class CLConv:
    """One conv of the decoder with its packed weights, bias, snake vectors and per-row state
    (_CLConv, fast_engine.py:178-233). weight / bias are the module's tensors; alpha the snake's [Cin] (or
    None); dilation for a Conv1d, stride for a ConvTranspose1d (trans=True). tmax: the most input rows a call
    takes (a frame's length at this conv); the split-K workspace is sized once for every row count up to Bmax
    at tmax rows. A call with more rows or a shape needing more runs K unsplit (nothing is allocated in a
    call)."""

    def __init__(self, weight, bias, Bmax, dev, states, alpha=None, trans=False, stride=1, dilation=1, tmax=None):
        self.W, self.taps, self.ph = pack_conv(weight.to(dev), trans, stride)
        self.dil = 1 if trans else int(dilation)
        self.ctx = 1 if trans else (self.taps - 1) * self.dil
        self.Cin, self.Cout = (weight.shape[0], weight.shape[1]) if trans else (weight.shape[1], weight.shape[0])
        self.bias = bias.detach().to(dev, F16).contiguous() if bias is not None else None
        self.a = self.ib = None
        if alpha is not None:
            al = alpha.detach().to(dev, torch.float32).reshape(-1)
            self.a = al.contiguous()
            self.ib = (1.0 / (al + 1e-9)).contiguous()
        self.state = None
        if self.ctx > 0:
            self.state = torch.zeros(Bmax, self.ctx, self.Cin, dtype=F16, device=dev)
            states.append(self.state)
        self.ws = None
        if tmax and torch.device(dev).type == "cuda":
            need = max(conv_cl_ws_bytes(b, int(tmax), self.Cin, self.Cout, self.taps, self.ph)
                       for b in range(1, Bmax + 1))
            if need > 0:
                self.ws = torch.empty(need, dtype=torch.uint8, device=dev)

    def __call__(self, x, b, res=None):
        """x [b, T, Cin] fp16 (pre-activation) -> [b, T*ph, Cout] fp16."""
        T = x.shape[1]
        y = torch.empty(b, T * self.ph, self.Cout, dtype=F16, device=x.device)
        if self.state is None:
            snake = (self.a, self.ib) if self.a is not None else None
            conv_cl(x.contiguous(), self.W, self.bias, T, self.taps, self.dil, self.ph, y, res=res, snake=snake,
                    ws=self.ws)
            return y
        xin = torch.empty(b, self.ctx + T, self.Cin, dtype=F16, device=x.device)
        refresh = T >= self.ctx  # the next context written by snake_cat itself (no copy after the conv)
        snake_cat(x, self.state[:b], self.a, self.ib, xin, refresh=refresh)
        conv_cl(xin, self.W, self.bias, T, self.taps, self.dil, self.ph, y, res=res, ws=self.ws)
        if not refresh:
            self.state[:b].copy_(xin[:, T:])
        return y


class FusedRU:
    """A residual unit (snake, causal conv k dil, snake, conv 1x1, + input) as one launch after the state concat
    (the reference's _FusedRU, fast_engine.py:235-273, on ru_cl): the k-tap conv's output stays in registers
    (fp32, the second snake applied there, one rounding to fp16) and feeds the 1x1 conv in the same workgroup.
    Uses c1's state (activated context) and refreshes it after, as the two-conv path does (any chunk length).
    Widths 96, 192 and 384 (RU_WIDTHS): one workgroup tile holds a row's channels."""

    RU_WIDTHS = (96, 192, 384)
    # the widths the decoder fuses by default: at 384 channels the fused unit measured slower than the two convs
    # (201 vs 190 us at block 1's 49152 rows: one row tile and 32-channel slices to fit the row's 384 channels)
    DEFAULT_WIDTHS = (96, 192)

    def __init__(self, c1, c2):
        assert c1.Cin == c1.Cout == c2.Cin == c2.Cout and c2.taps == 1 and c1.ph == c2.ph == 1
        assert c1.state is not None and c1.a is not None and c2.a is not None
        assert c1.Cin in self.RU_WIDTHS and c1.bias is not None and c2.bias is not None
        self.c1, self.c2 = c1, c2
        self.w1 = c1.W[0]            # [taps, C, C]
        self.w2 = c2.W[0, 0]         # [C, C]

    def __call__(self, x, b):
        c1, c2 = self.c1, self.c2
        T = x.shape[1]
        xin = torch.empty(b, c1.ctx + T, c1.Cin, dtype=F16, device=x.device)
        refresh = T >= c1.ctx
        snake_cat(x, c1.state[:b], c1.a, c1.ib, xin, refresh=refresh)
        y = torch.empty(b, T, c1.Cout, dtype=F16, device=x.device)
        ru_cl(xin, self.w1, c1.bias, c2.a, c2.ib, self.w2, c2.bias, x, y, T, c1.taps, c1.dil)
        if not refresh:
            c1.state[:b].copy_(xin[:, T:])
        return y


def decoder_weights(cin=1024, ch=1536, rates=(8, 8, 4, 2), k=7, dils=(1, 3, 9), dev="cpu", seed=0):
    """A synthetic decoder in the modules' own layouts: conv_in (w [ch, cin, k], b), blocks of (alpha, transposed
    w [C, C/2, 2s], b, stride, units of (alpha1, w1 [C/2, C/2, k], b1, dil, alpha2, w2 [C/2, C/2, 1], b2)),
    final (alpha, w [1, C_last, k], b). Weights ~ N(0, 1/fan_in), snake alphas ~ U[0.5, 1.5]."""
    g = torch.Generator(device="cpu").manual_seed(seed)

    def conv(co, ci, kk, fan):
        return (torch.randn(co, ci, kk, generator=g) / fan ** 0.5).to(dev), (0.02 * torch.randn(co, generator=g)).to(dev)

    def alpha(c):
        return (0.5 + torch.rand(c, generator=g)).to(dev)

    wts = {"conv_in": conv(ch, cin, k, cin * k), "blocks": []}
    C = ch
    for s in rates:
        tw = (torch.randn(C, C // 2, 2 * s, generator=g) / (C * 2) ** 0.5).to(dev)
        tb = (0.02 * torch.randn(C // 2, generator=g)).to(dev)
        a0 = alpha(C)
        C //= 2
        units = []
        for d in dils:
            w1, b1 = conv(C, C, k, C * k)
            w2, b2 = conv(C, C, 1, C)
            units.append((alpha(C), w1, b1, d, alpha(C), w2, b2))
        wts["blocks"].append((a0, tw, tb, s, units))
    wf, bf = conv(1, C, k, C * k)
    wts["final"] = (alpha(C), wf, bf)
    return wts


class CLDecoder:
    """The stateful channels-last decoder (_CLDecoder, fast_engine.py:276-310) over `decoder_weights`-shaped
    weights; every conv's state is registered in `states` (per row, for snapshots / row resets). frame: the
    input rows a call takes (sizes each conv's split-K workspace once; the streaming decoder's frame is 4)."""

    def __init__(self, wts, Bmax, dev, states=None, frame=4, fused_ru=()):
        self.states = states if states is not None else []
        fuse = set(int(c) for c in (fused_ru or ()))
        S = self.states
        w, b = wts["conv_in"]
        t = int(frame)
        self.dec_in = CLConv(w, b, Bmax, dev, S, dilation=1, tmax=t)
        self.blocks = []
        for a0, tw, tb, s, units in wts["blocks"]:
            tc = CLConv(tw, tb, Bmax, dev, S, alpha=a0, trans=True, stride=s, tmax=t)
            t *= s
            us = []
            for a1, w1, b1, d, a2, w2, b2 in units:
                c1 = CLConv(w1, b1, Bmax, dev, S, alpha=a1, dilation=d, tmax=t)
                c2 = CLConv(w2, b2, Bmax, dev, S, alpha=a2, tmax=t)
                fu = FusedRU(c1, c2) if (c1.Cin in fuse and c1.Cin in FusedRU.RU_WIDTHS and
                                         torch.device(dev).type == "cuda") else None
                us.append((c1, c2, fu))
            self.blocks.append((tc, us))
        af, wf, bf = wts["final"]
        self.final = CLConv(wf, bf, Bmax, dev, S, alpha=af, tmax=t)
        # fused_out: the last conv (one channel) as one launch with its snake_cat, state refresh and tanh
        # (conv_out_tanh), where its shape allows; else snake_cat + conv_cl + the state copy + tanh
        f = self.final
        self.wout = f.W[0, :, :, 0].contiguous()  # [taps, Cin]: the one output channel's weights
        self.fused_out = (f.Cout == 1 and f.ph == 1 and f.dil == 1 and f.state is not None and f.Cin % 8 == 0
                          and f.Cin <= 128 and f.taps <= 8)
        self.up = 1
        for _, _, _, s, _ in wts["blocks"]:
            self.up *= s

    def reset_rows(self, rows):
        """Zero the state of the given rows (a new utterance starts from silence)."""
        for st in self.states:
            st[rows] = 0

    def __call__(self, x, b):
        """x [b, T, cin] -> wav [b, T * up] float32 (tanh)."""
        x = self.dec_in(x.to(F16).contiguous(), b)
        for tc, units in self.blocks:
            x = tc(x, b)
            for c1, c2, fu in units:
                x = fu(x, b) if fu is not None else c2(c1(x, b), b, res=x)
        f = self.final
        if self.fused_out and x.shape[1] >= f.ctx:
            y = torch.empty(b, x.shape[1], dtype=torch.float32, device=x.device)
            return conv_out_tanh(x.contiguous(), f.state[:b], f.a, f.ib, self.wout, f.bias, y)
        return f(x, b)[..., 0].float().tanh()
