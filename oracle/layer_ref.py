"""CPU oracle for the slow-AR layer steps around the attention path.

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker; the product path never calls it.

Restates, in torch on the CPU with the reference's roundings (bf16 storage, fp32 math):

    rmsnorm     serve/fast_kernels.py:30-69 (_rmsnorm_kernel, rmsnorm): optional bf16 residual add,
                fp32 mean of squares, xn rounded to bf16, weight * xn rounded to bf16
    silu_mul    serve/fast_kernels.py:526-545 (_silu_mul_kernel, silu_mul): bf16(silu(g)) * u in bf16
    linear      fast_engine.py:90 (the default mm, torch.matmul(x, w.t())): bf16 operands, fp32
                accumulation, one bf16 rounding
    slow_stack  serve/fast_engine.py:117-138 (_Stack.forward) on attn_ref's store / decode / prefill

Pinned by tests/test_oracle.py against library routines and closed forms, not by retyping: rmsnorm
against torch.nn.functional.rms_norm in float64 (then the same two roundings), silu_mul against
torch.nn.functional.silu, linear against a float64 matmul, slow_stack's residual stream against a
hand-unrolled one-layer float64 evaluation.
"""
from __future__ import annotations

import torch

from . import attn_ref

BF16 = torch.bfloat16


def rmsnorm(x, w, eps, residual=None):
    """(y, h) with h = bf16(x + residual) (or x), y = bf16(w * bf16(h * rsqrt(mean(h^2) + eps)))
    (fast_kernels.py:30-46)."""
    h = (x.float() + residual.float()).to(BF16) if residual is not None else x
    hf = h.float()
    var = (hf * hf).sum(-1, keepdim=True) / hf.shape[-1]
    xn = (hf * torch.rsqrt(var + eps)).to(BF16)
    y = (w.float() * xn.float()).to(BF16)
    return y, h


def silu_mul(gu):
    """gu [..., 2I] -> bf16(bf16(g / (1 + exp(-g))) * u) (fast_kernels.py:526-534)."""
    I = gu.shape[-1] // 2
    g, u = gu[..., :I].float(), gu[..., I:].float()
    gs = (g / (1.0 + torch.exp(-g))).to(BF16).float()
    return (gs * u).to(BF16)


def linear(x, w):
    """x [M, K] @ w[N, K]^T with fp32 accumulation, rounded once to bf16 (the default mm of
    fast_engine.py:90, a cuBLAS / hipBLASLt bf16 GEMM)."""
    return (x.float() @ w.float().t()).to(BF16)


def slow_stack(x, pos, slot, lens, layers, norm, nq, nkv, hd, eps, cos, sin, kc, vc, rowmap=True, plan=None,
               ring=1 << 30):
    """_Stack.forward (fast_engine.py:117-138) on CPU tensors. layers: list of dicts wqkv, bqkv, wo, w13, w2,
    ln1, ln2; kc / vc: per-layer caches, updated in place. plan: (q0s, ns, slots, p0s) for the packed
    prefill, else the decode with lens (rowmap = slot when rowmap). Returns the final-normed hidden."""
    R = x.shape[0]
    nl = len(layers)
    h, _ = rmsnorm(x, layers[0]["ln1"], eps)
    res = x
    for i, L in enumerate(layers):
        qkv = linear(h, L["wqkv"])
        q = torch.zeros(R, nq, hd, dtype=BF16)
        attn_ref.bias_rope_store(qkv, L["bqkv"], cos, sin, pos, slot, q, kc[i], vc[i], nq, nkv, hd, ring=ring)
        if plan is not None:
            o = torch.zeros(R, nq, hd, dtype=BF16)
            attn_ref.prefill_attention(q, kc[i], vc[i], *plan, o, nq // nkv)
        else:
            o = attn_ref.decode_attention(q, kc[i], vc[i], lens, rowmap=slot if rowmap else None)
        a = linear(o.reshape(R, -1), L["wo"])
        h, res = rmsnorm(a, L["ln2"], eps, residual=res)
        m = linear(silu_mul(linear(h, L["w13"])), L["w2"])
        nxt = layers[i + 1]["ln1"] if i + 1 < nl else norm
        h, res = rmsnorm(m, nxt, eps, residual=res)
    return h
