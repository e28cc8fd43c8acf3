"""CPU oracle for the streaming vocoder's channels-last convolutions.

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker; the product path never calls it.

Restates, in torch on the CPU (fp16 storage, fp32 math):

    snake      serve/fast_kernels.py:571-575 / 709-712 (the snake on a load): x + ib sin(a x)^2, one fp16 rounding
    conv_cl    serve/fast_kernels.py:551-623 (_conv_cl_kernel, conv_cl): out[b, t*ph + p] = bias
               + sum_j x[b, t + j*dil] @ w[p, j] (+ res[b, t*ph + p]), fp32 accumulation, one fp16 rounding
    snake_cat  serve/fast_kernels.py:695-729 (_snake_cat_kernel, snake_cat): concat(state, snake(x)) in time
    ru_fused   serve/fast_kernels.py:626-692 (_ru_fused_kernel, ru_fused): a whole residual unit, h kept fp32
    decoder    serve/fast_engine.py:276-310 (_CLDecoder) over a whole utterance from silence, written directly
               on torch's conv1d / conv_transpose1d of the modules' own weights (channels first, float64,
               rounded to fp16 where the channels-last path stores: the snake's output and each conv's output)

Pinned by tests/test_oracle.py against torch.nn.functional.conv1d (causal / dilated, ph = 1) and
conv_transpose1d (the phase split of a stride-s transposed conv, as fast_engine.py:186-194 builds it), in
float64, and by a brute-force loop on tiny sizes; ru_fused against the two-conv unit (snake_cat, conv_cl,
conv_cl with the residual) bit for bit where the second snake is the identity (ib2 = 0: h rounds to fp16
either way), and against a float64 loop with the snake; decoder's composition (block order, transposed-conv
crop, unit order and dilations, causal taps) against the closed-form impulse response of structured weights
(identity snakes, delta taps, sample-repeat transposed convs), and by a causality invariant on random weights.
"""
from __future__ import annotations

import torch

F16 = torch.float16


def snake(x, a, ib):
    """x + ib * sin(a * x)^2 in fp32, rounded to fp16 (channels last: a / ib broadcast over the last dim)."""
    xf = x.float()
    s = torch.sin(xf * a.float())
    return (xf + ib.float() * s * s).to(F16)


def conv_cl(xin, w, bias, TR, taps, dil, ph, Cout, res=None, snake_ab=None):
    """out [B, TR*ph, Cout] fp16 from xin [B, Tin, Cin], w [ph, taps, Cin, >=Cout] (fast_kernels.py:551-597)."""
    B = xin.shape[0]
    x = snake(xin, *snake_ab).float() if snake_ab is not None else xin.float()
    out = torch.empty(B, TR * ph, Cout, dtype=torch.float32)
    for p in range(ph):
        acc = torch.zeros(B, TR, Cout, dtype=torch.float32)
        for j in range(taps):
            acc += x[:, j * dil:j * dil + TR, :] @ w[p, j, :, :Cout].float()
        if bias is not None:
            acc += bias[:Cout].float()
        if res is not None:
            acc += res[:, p::ph][:, :TR, :Cout].float()
        out[:, p::ph] = acc
    return out.to(F16)


def snake_cat(x, state, a, ib):
    """concat(state (CTX activated rows), snake(x) (T rows)) along time (fast_kernels.py:695-715)."""
    y = snake(x, a, ib) if a is not None else x
    return torch.cat([state, y], 1) if state is not None else y


def ru_fused(x, state, a1, ib1, w1, b1, a2, ib2, w2, b2, taps, dil):
    """One whole residual unit (fast_kernels.py:626-692, _ru_fused_kernel / ru_fused; _FusedRU, fast_engine.py
    :235-273): out = x + b2 + snake2(b1 + conv_k(snake1([state | x]), dil)) @ w2, channels last.
    x [B, T, C] raw fp16, state [B, CTX, C] activated (CTX = (taps - 1) dil), w1 [taps, C, C] and w2 [C, C] fp16
    [k][n], b1 / b2 fp16 [C], a1 / ib1 / a2 / ib2 fp32 [C]. The first conv's output h = acc + b1 stays fp32; the
    second snake runs on it in fp32 and rounds once to fp16 (fast_kernels.py:659-663); sums in fp32 (the
    reference's F16ACC fp16 partial sums are the less exact variant and are not modelled)."""
    xin = snake_cat(x, state, a1, ib1).float()
    B, T, C = x.shape
    h = torch.zeros(B, T, C, dtype=torch.float32)
    for j in range(taps):
        h += xin[:, j * dil:j * dil + T, :] @ w1[j].float()
    h += b1[:C].float()
    s = torch.sin(h * a2[:C].float())
    hf = (h + ib2[:C].float() * s * s).to(F16).float()
    out = hf @ w2.float()
    out += b2[:C].float()
    out += x.float()
    return out.to(F16)


def _f16(t):
    return t.to(F16).double()


def _conv_fc(x, w, b, dil=1, alpha=None, res=None, trans=False, stride=1):
    """One causal conv over a whole utterance, channels first x [B, C, T] (fp16 values, float64 storage):
    snake (rounded to fp16), zero left context, conv in float64 with fp16-rounded weights and bias, + res,
    rounded to fp16."""
    if alpha is not None:
        a = alpha.double().view(1, -1, 1)
        s = torch.sin(a.float() * x.float()).double()
        x = _f16(x + (1.0 / (a.float() + 1e-9)).double() * s * s)
    W, bb = _f16(w), _f16(b) if b is not None else None
    if trans:
        T = x.shape[-1]
        y = torch.nn.functional.conv_transpose1d(x, W, bb, stride=stride)[..., :T * stride]
    else:
        ctx = (w.shape[-1] - 1) * dil
        y = torch.nn.functional.conv1d(torch.nn.functional.pad(x, (ctx, 0)), W, bb, dilation=dil)
    if res is not None:
        y = y + res
    return _f16(y)


def decoder(wts, x):
    """wts as vocoder.decoder_weights builds them (the modules' tensors); x [B, T, cin] -> wav [B, T * up]
    float64 (tanh of the fp16 output), the whole utterance from zero state (fast_engine.py:302-310)."""
    h = _conv_fc(_f16(x.transpose(1, 2)), *wts["conv_in"])
    for a0, tw, tb, s, units in wts["blocks"]:
        h = _conv_fc(h, tw, tb, alpha=a0, trans=True, stride=s)
        for a1, w1, b1, d, a2, w2, b2 in units:
            h = _conv_fc(_conv_fc(h, w1, b1, dil=d, alpha=a1), w2, b2, alpha=a2, res=h)
    af, wf, bf = wts["final"]
    return torch.tanh(_conv_fc(h, wf, bf, alpha=af)[:, 0])
