"""CPU oracle: a torch-CPU restatement of the reference's attention hot path.

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker (or as the timed CPU baseline); the product path never calls it.

It restates, step for step, the semantics of lvt1693/audio8-turbo-engine's Triton kernels and their
callers, keeping the reference's numerics: bf16 storage, fp32 math, q/k rotated then rounded once to
bf16, online softmax in fp32 over 64-key tiles with the softmax weights rounded to bf16 before the
P.V product (fp32 accumulate), and the split/combine structure of the decode path.

    rope_tables        serve/fast_engine.py:70-75
    permute_qk         serve/fast_engine.py:60-67
    bias_rope_store    serve/fast_kernels.py:139-187
    decode_attention   serve/fast_kernels.py:193-290 (split kernel 193-235, combine 238-253, call 271-290)
    ref_nsplit         serve/fast_engine.py:776
    prefill_plan       serve/fast_kernels.py:335-347
    pf_meta_host       serve/fast_engine.py:837-853
    prefill_attention  serve/fast_kernels.py:296-358

Every function is pinned by checks in tests/test_oracle.py that do not retype it: numpy float64
closed forms (RoPE tables, rotation, softmax attention), an independent numpy float32 / bf16-rounding
implementation of the store (bit-exact), brute-force index coverage (store slots, plans), invariants
(q.k preserved by the permutation, split-count independence, L=1 and constant-key special cases,
key-permutation invariance, prefill row == decode at lens = pos+1) and the committed golden vectors in
tests/golden/ (written by tests/golden/make_golden.py from float64 numpy, not from this file).
"""
from __future__ import annotations

import math

import numpy as np
import torch

BF16 = torch.bfloat16
NEG_INF = float("-inf")


def _cdiv(a, b):
    return -(-a // b)


# ----------------------------------------------------------------------------------------------
# a1 / a2: RoPE tables and the interleaved -> rotate_half permutation
# ----------------------------------------------------------------------------------------------
def rope_tables(base, hd, n):
    """cos / sin [n, hd] bf16: fp32 phase pos * base^(-2i/hd), rounded to bf16, duplicated [c, c]
    (fast_engine.py:70-75)."""
    fr = 1.0 / (base ** (torch.arange(0, hd, 2).float()[: hd // 2] / hd))
    ph = torch.outer(torch.arange(n).float(), fr)
    c, s = ph.cos().to(BF16), ph.sin().to(BF16)
    return torch.cat([c, c], -1), torch.cat([s, s], -1)


def permute_qk(w, nq, nkv, hd):
    """Fused-projection rows with q / k head dims reordered (2i, 2i+1) -> (i, i+hd/2) (fast_engine.py:60-67)."""
    p = torch.cat([torch.arange(0, hd, 2), torch.arange(1, hd, 2)])
    rest = w.shape[1:]
    q = w[:nq * hd].reshape(nq, hd, *rest)[:, p].reshape(nq * hd, *rest)
    k = w[nq * hd:(nq + nkv) * hd].reshape(nkv, hd, *rest)[:, p].reshape(nkv * hd, *rest)
    return torch.cat([q, k, w[(nq + nkv) * hd:]], 0)


# ----------------------------------------------------------------------------------------------
# a3: qkv bias + rotate_half RoPE + KV store
# ----------------------------------------------------------------------------------------------
def bias_rope_store(qkv, bias, cos_tab, sin_tab, pos, slot, qo, kc, vc, nq, nkv, hd, ring=1 << 30):
    """In place on CPU tensors, like fast_kernels.py:139-187: qo[r] <- rotated q, kc / vc[slot, :, pos % ring]
    <- rotated k / biased v. The store order over rows is the row order (later rows win on collisions)."""
    R = qkv.shape[0]
    if R == 0:
        return qo
    H = nq + 2 * nkv
    half = hd // 2
    d = torch.arange(hd)
    dp = (d + half) % hd
    sign = torch.where(d < half, -1.0, 1.0)
    x = qkv[:, :H * hd].float().view(R, H, hd)
    if bias is not None:
        x = x + bias[:H * hd].float().view(1, H, hd)
    p = pos.long()
    c = cos_tab[p, :hd].float().view(R, 1, hd)
    s = sin_tab[p, :hd].float().view(R, 1, hd)
    xqk = x[:, :nq + nkv]
    o = (xqk * c + sign * xqk[:, :, dp] * s).to(BF16)           # fast_kernels.py:167-172
    qo[:R] = o[:, :nq]
    sidx = torch.fmod(p, ring)                                      # Triton's % on int32 (C remainder)
    sl = slot.long()                                                # fast_kernels.py:153
    for r in range(R):                                              # row order: deterministic on collisions
        kc[sl[r], :, sidx[r]] = o[r, nq:]
        vc[sl[r], :, sidx[r]] = x[r, nq + nkv:].to(BF16)            # fast_kernels.py:157-162
    return qo


# ----------------------------------------------------------------------------------------------
# a5-a8: split-K decode attention
# ----------------------------------------------------------------------------------------------
def ref_nsplit(b, nkv):
    """fast_engine.py:776."""
    return max(1, min(16, -(-2 * 84 // (b * nkv))))


def decode_split(q, kc, vc, lens, nsplit, rowmap=None, scale=None, bn=64):
    """The split kernel (fast_kernels.py:193-235), vectorised over rows and kv heads.
    Returns acc [b, nq, nsplit, hd] fp32 and ml [b, nq, nsplit, 2] fp32 (m, l) with m in natural units."""
    b, nq, hd = q.shape
    nkv, S = kc.shape[1], kc.shape[2]
    group = nq // nkv
    scale = hd ** -0.5 if scale is None else scale
    acc = torch.zeros(b, nq, nsplit, hd)
    ml = torch.zeros(b, nq, nsplit, 2)
    if b == 0:
        return acc, ml
    L = lens[:b].long()
    crow = rowmap[:b].long() if rowmap is not None else torch.arange(b)
    per = ((L + nsplit - 1) // nsplit + bn - 1) // bn * bn               # cdiv(cdiv(L, NSPLIT), BN) * BN
    qg = q.float().view(b, nkv, group, hd)
    ar = torch.arange(bn)
    for sp in range(nsplit):
        lo = sp * per
        hi = torch.minimum(lo + per, L)
        m = torch.full((b, nkv, group), NEG_INF)
        l = torch.zeros(b, nkv, group)
        a = torch.zeros(b, nkv, group, hd)
        ntile = int(((hi - lo).clamp(min=0) + bn - 1).div(bn, rounding_mode="floor").max())
        for t in range(ntile):
            start = lo + t * bn                                           # [b]
            active = start < hi                                           # rows with this tile
            n = start[:, None] + ar[None, :]                              # [b, bn]
            nm = n < hi[:, None]
            idx = n.clamp(0, S - 1)
            k = kc[crow[:, None], :, idx].float().permute(0, 2, 1, 3)     # [b, nkv, bn, hd]
            v = vc[crow[:, None], :, idx].float().permute(0, 2, 1, 3)
            k = torch.where(nm[:, None, :, None], k, 0.0)                 # masked loads read 0.0
            v = torch.where(nm[:, None, :, None], v, 0.0)
            s = torch.matmul(qg, k.transpose(-1, -2)) * scale             # [b, nkv, group, bn]
            s = torch.where(nm[:, None, None, :], s, torch.tensor(NEG_INF))
            m_new = torch.maximum(m, s.amax(-1))
            alpha = torch.exp(m - m_new)
            p = torch.exp(s - m_new[..., None])
            l_new = l * alpha + p.sum(-1)
            a_new = a * alpha[..., None] + torch.matmul(p.to(BF16).float(), v)
            act = active[:, None, None]
            m = torch.where(act, m_new, m)
            l = torch.where(act, l_new, l)
            a = torch.where(act[..., None], a_new, a)
        acc[:, :, sp] = a.reshape(b, nq, hd)
        ml[:, :, sp, 0] = m.reshape(b, nq)
        ml[:, :, sp, 1] = l.reshape(b, nq)
    return acc, ml


def decode_combine(acc, ml, out_dtype=BF16):
    """The combine kernel (fast_kernels.py:238-253): out = sum(w acc) / sum(w l), w = exp(m - M), stored in
    the output's dtype (bf16, or fp32 for an fp32 output; fast_kernels.py:253)."""
    m, l = ml[..., 0], ml[..., 1]
    M = m.amax(-1, keepdim=True)
    w = torch.where(m == NEG_INF, torch.zeros(()), torch.exp(m - M))
    num = (acc * w[..., None]).sum(-2)
    den = (l * w).sum(-1)
    return (num / den[..., None]).to(out_dtype)


def decode_attention(q, kc, vc, lens, nsplit=1, rowmap=None, scale=None, bn=64, out_dtype=BF16):
    """DecodeAttention.__call__ (fast_kernels.py:271-290) on CPU tensors; returns out [b, nq, hd] (bf16, or
    out_dtype). q may be bf16 or fp32: the split works on q.float() either way, which is the reference's
    PREC = "ieee" product for an fp32 q (fast_kernels.py:279) and exact for a bf16 one."""
    acc, ml = decode_split(q, kc, vc, lens, max(1, int(nsplit)), rowmap, scale, bn)
    return decode_combine(acc, ml, out_dtype)


# ----------------------------------------------------------------------------------------------
# a9-a11: packed prefill
# ----------------------------------------------------------------------------------------------
BM = 64


def prefill_plan(r0s, ns, slots, p0s):
    """PrefillPlan's block lists (fast_kernels.py:335-347): (q0, n, slot, pos0) per <= 64-row block."""
    q0, cnt, sl, ps = [], [], [], []
    for r0, n, s, p0 in zip(r0s, ns, slots, p0s):
        for off in range(0, n, BM):
            q0.append(r0 + off)
            cnt.append(min(BM, n - off))
            sl.append(s)
            ps.append(p0 + off)
    return q0, cnt, sl, ps


def pf_layout(NT, NR):
    """Offsets of the graph-mode plan buffer [pos NT | slot NT | q0, n, bslot, pos0 NB | last, st, cpos NR]
    (fast_engine.py:684-691)."""
    NB = NT // BM + NR
    return np.cumsum([0, NT, NT, NB, NB, NB, NB, NR, NR, NR])


def pf_meta_host(nt, slots, ns, starts, NT, NR, SCR):
    """fast_engine.py:837-853: int32 plan of requests of ns tokens at positions starts.. in slots."""
    o = pf_layout(NT, NR)
    m = np.zeros(int(o[-1]), np.int32)
    pos, slot, q0, n, bslot, p0, last, st, cpos = (m[o[i]:o[i + 1]] for i in range(9))
    slot[:], bslot[:], st[:] = SCR, SCR, SCR
    r0 = bi = 0
    for k, (s, cnt, a) in enumerate(zip(slots, ns, starts)):
        pos[r0:r0 + cnt] = np.arange(a, a + cnt)
        slot[r0:r0 + cnt] = s
        for off in range(0, cnt, BM):
            q0[bi], n[bi], bslot[bi], p0[bi] = r0 + off, min(BM, cnt - off), s, a + off
            bi += 1
        last[k], st[k], cpos[k] = r0 + cnt - 1, s, a + cnt
        r0 += cnt
    assert r0 <= nt and bi <= nt // BM + NR and len(slots) <= NR
    return m


def prefill_attention(q, kc, vc, q0s, ns, slots, p0s, out, group, scale=None, bn=64):
    """The prefill kernel (fast_kernels.py:296-332) over a block plan (lists or int tensors), in place on
    out [R, nq, hd] bf16. Each block: rows q0..q0+n-1 at positions p0.., keys [0, p0+n) of cache row slot,
    mask key <= query position, 64-key tiles, online softmax in fp32, P rounded to bf16, out = bf16(acc/l)."""
    nq, hd = q.shape[1], q.shape[2]
    nkv = nq // group
    scale = hd ** -0.5 if scale is None else scale
    kv_of = torch.arange(nq) // group
    for q0, n, slot, p0 in zip(*(list(map(int, x)) for x in (q0s, ns, slots, p0s))):
        if n <= 0:
            continue
        qb = q[q0:q0 + n].float().permute(1, 0, 2)                        # [nq, n, hd]
        qpos = p0 + torch.arange(n)
        hi = p0 + n
        m = torch.full((nq, n), NEG_INF)
        l = torch.zeros(nq, n)
        a = torch.zeros(nq, n, hd)
        for start in range(0, hi, bn):
            kn = start + torch.arange(bn)
            nm = kn < hi
            idx = kn.clamp(max=hi - 1)
            k = torch.where(nm[None, :, None], kc[slot][:, idx].float(), 0.0)   # [nkv, bn, hd]; masked -> 0
            v = torch.where(nm[None, :, None], vc[slot][:, idx].float(), 0.0)
            s = torch.matmul(qb, k[kv_of].transpose(-1, -2)) * scale      # [nq, n, bn]
            valid = (kn[None, :] <= qpos[:, None]) & nm[None, :]
            s = torch.where(valid[None], s, torch.tensor(NEG_INF))
            m_new = torch.maximum(m, s.amax(-1))
            alpha = torch.exp(m - m_new)
            p = torch.exp(s - m_new[..., None])
            l = l * alpha + p.sum(-1)
            a = a * alpha[..., None] + torch.matmul(p.to(BF16).float(), v[kv_of])
            m = m_new
        out[q0:q0 + n] = (a / l[..., None]).permute(1, 0, 2).to(BF16)
    return out


def decode_bytes(lens, nq, nkv, hd, with_store=True, width=None):
    """Algorithmic HBM bytes of one layer of store + decode for rows with the given key lengths:
    K+V read (lens * nkv * hd * 2 * 2 B) + q in + out, plus the store's qkv read, q write, k/v write,
    pos/slot, bias and cos/sin rows."""
    b = len(lens)
    kv = int(sum(int(x) for x in lens)) * nkv * hd * 2 * 2
    qo = 2 * b * nq * hd * 2
    total = kv + qo
    if with_store:
        width = (nq + 2 * nkv) * hd if width is None else width
        # cos / sin rows counted as b * 2 * hd * 2 * 2 B, the figure the 203.0 MB/layer C3 target uses
        total += b * (width * 2 + nq * hd * 2 + 2 * nkv * hd * 2 + 8) + width * 2 + b * 2 * hd * 2 * 2
    return total


def prefill_flops(ns, p0s, nq, hd):
    """Algorithmic FLOPs of causal prefill (unmasked pairs only): 4 * nq * hd * sum_i sum_j (p0_i + j + 1)."""
    pairs = 0
    for n, p0 in zip(ns, p0s):
        pairs += n * (p0 + 1) + n * (n - 1) // 2
    return 4 * nq * hd * pairs


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("annotations", "math", "np", "torch")]
