"""a2 on the device: permute_qk (fast_engine.py:60-67) applied to weights and biases resident on the GPU equals the
CPU oracle bit for bit, and, fed through the device store kernel (rotate_half RoPE), gives the q . k scores of
the checkpoint's interleaved RoPE on the unpermuted projection (float64 textbook) within bf16 rounding."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
NQ, NKV, HD, HID = 14, 2, 64, 896
W = (NQ + 2 * NKV) * HD


def _interleaved_rope(x, pos, base, hd):
    """Textbook interleaved RoPE on the last axis: pairs (2i, 2i+1) rotated by pos * base^(-2i/hd)."""
    i = np.arange(hd // 2)
    th = pos * base ** (-2.0 * i / hd)
    c, s = np.cos(th), np.sin(th)
    a, b = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = a * c - b * s
    out[..., 1::2] = a * s + b * c
    return out


def test_permute_qk_on_device(a8, ref):
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(W, HID, generator=g) * 0.05).to(BF)
    bias = (torch.randn(W, generator=g) * 0.02).to(BF)
    print("case: permute_qk [1152, 896] weight and [1152] bias on cuda:0", flush=True)
    wp_d, bp_d = a8.permute_qk(w.to(dev), NQ, NKV, HD), a8.permute_qk(bias.to(dev), NQ, NKV, HD)
    torch.cuda.synchronize()
    assert wp_d.is_cuda and bp_d.is_cuda
    assert torch.equal(wp_d.cpu(), ref.permute_qk(w, NQ, NKV, HD)), "weight rows"
    assert torch.equal(bp_d.cpu(), ref.permute_qk(bias, NQ, NKV, HD)), "bias"

    # the permuted projection through the device store kernel == interleaved RoPE on the original projection
    R, S = 4, 2048
    x = torch.randn(R, HID, generator=g, dtype=torch.float64)
    qkv_il = x @ w.double().T                                    # checkpoint layout (interleaved pairs)
    qkv_rh = (x @ wp_d.cpu().double().T).to(BF)                  # permuted rows: rotate_half layout
    pos = torch.tensor([0, 7, 1234, 2047], dtype=torch.int32)
    slot = torch.arange(R, dtype=torch.int32)
    cos, sin = a8.rope_tables(10000.0, HD, S, dev)
    qo = torch.empty(R, NQ, HD, dtype=BF, device=dev)
    kc = torch.zeros(R, NKV, S, HD, dtype=BF, device=dev)
    vc = torch.zeros_like(kc)
    a8.bias_rope_store(qkv_rh.to(dev), bp_d, cos, sin, pos.to(dev), slot.to(dev), qo, kc, vc, NQ, NKV, HD)
    torch.cuda.synchronize()
    q_dev = qo.cpu().double().numpy()
    b64 = bias.double().numpy()
    worst = 0.0
    for r in range(R):
        p = int(pos[r])
        k_dev = kc[r, :, p].cpu().double().numpy()               # [NKV, HD]
        for h in range(NQ):
            kh = h // (NQ // NKV)
            qi = _interleaved_rope(qkv_il[r, h * HD:(h + 1) * HD].numpy() + b64[h * HD:(h + 1) * HD], p, 10000.0, HD)
            kb = (NQ + kh) * HD
            ki = _interleaved_rope(qkv_il[r, kb:kb + HD].numpy() + b64[kb:kb + HD], p, 10000.0, HD)
            want = float(qi @ ki)
            got = float(q_dev[r, h] @ k_dev[kh])
            # bf16 qkv, tables and outputs: the oracle's store on the same inputs lands within 0.011 of
            # |q| |k| / sqrt(hd) (6 seeds); without the permutation the error is of order 1
            tol = 4e-2 * (np.linalg.norm(qi) * np.linalg.norm(ki)) / np.sqrt(HD)
            worst = max(worst, abs(want - got) / tol)
            assert abs(want - got) <= tol, (r, h, want, got)
    print(f"permute_qk on device: scores within {worst:.2f} of the bf16 tolerance", flush=True)
