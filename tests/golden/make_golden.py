"""Writes the golden vectors in this directory. Run from the repository root:

    python tests/golden/make_golden.py

The reference (lvt1693/audio8-turbo-engine) ships no test vectors for its attention path, so these are
computed here from the mathematics of that path with numpy alone -- neither the oracle (oracle/) nor the
product is imported -- and serve as an independent check of both:

  rope.npz     RoPE tables: cos / sin of pos * base^(-2i/hd) in float64, plus the fp32 phase the
               reference rounds from (fast_engine.py:70-75)
  store.npz    bias + rotate_half RoPE + KV store (fast_kernels.py:139-187): bf16 inputs, expected bf16
               outputs from numpy float32 arithmetic in the reference's operation order (two rounded
               products, one rounded sum) and round-to-nearest-even narrowing; a sentinel-filled cache
  decode.npz   GQA decode attention (fast_kernels.py:193-290): textbook softmax(q k^T / sqrt(hd)) v in
               float64 over keys [0, lens) of cache row rowmap[i]
  prefill.npz  packed causal prefill over a cached prefix (fast_kernels.py:296-358): per query row,
               float64 softmax over keys [0, its position] of its request's cache row (stored as
               float16: |error| <= 2.5e-4 for these outputs, far below the 2e-2 parity bound)

bf16 values are stored as uint16 bit patterns.
"""
from __future__ import annotations

import os

import numpy as np

OUT = os.path.dirname(os.path.abspath(__file__))


def f32_to_bf16_bits(x):
    """Round-to-nearest-even float32 -> bf16 bit pattern (NaN -> 0x7fc0)."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), r)


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def rand_bf16(rng, shape, std=1.0):
    return f32_to_bf16_bits((rng.standard_normal(shape) * std).astype(np.float32))


def rope(rng):
    base, hd, n = 10000.0, 64, 4096
    i = np.arange(hd // 2, dtype=np.float64)
    fr64 = base ** (-2.0 * i / hd)
    pos = np.unique(np.concatenate([np.arange(64), [64, 100, 127, 128, 255, 256, 300, 384, 511, 512, 1000,
                                                     1023, 1024, 2047, 2048, 3000, 4000, 4095]])).astype(np.float64)
    ph64 = np.outer(pos, fr64)
    # the reference's phase: fp32 inverse frequency times fp32 position, one fp32 rounding
    fr32 = (np.float32(1.0) / np.power(np.float32(base), np.arange(0, hd, 2, dtype=np.float32) / np.float32(hd)))
    ph32 = np.outer(pos.astype(np.float32), fr32.astype(np.float32)).astype(np.float32)
    np.savez_compressed(os.path.join(OUT, "rope.npz"), base=base, hd=hd, n=n, pos=pos.astype(np.int32),
                        cos64=np.cos(ph64).astype(np.float32), sin64=np.sin(ph64).astype(np.float32),
                        ph32=ph32)


def store(rng):
    nq, nkv, hd = 14, 2, 64
    H = nq + 2 * nkv
    W = H * hd
    rows, S, ring = 5, 40, 32
    R = 6
    qkv = rand_bf16(rng, (R, W))
    bias = rand_bf16(rng, (W,), 0.02)
    n_tab = 70
    cos_t = rand_bf16(rng, (n_tab, hd), 0.7)     # arbitrary tables: the store must use them as given
    sin_t = rand_bf16(rng, (n_tab, hd), 0.7)
    pos = np.array([0, 5, 31, 32, 45, 69], np.int32)        # 32, 45, 69 wrap the 32-slot ring
    slot = np.array([0, 4, 2, 1, 3, 0], np.int32)
    sentinel = np.uint16(0x7F7F)
    kc = np.full((rows, nkv, S, hd), sentinel, np.uint16)
    vc = np.full((rows, nkv, S, hd), sentinel, np.uint16)
    qo = np.full((R, nq, hd), sentinel, np.uint16)
    x = bf16_bits_to_f32(qkv).reshape(R, H, hd) + bf16_bits_to_f32(bias).reshape(1, H, hd)   # fp32 add
    d = np.arange(hd)
    partner = (d + hd // 2) % hd
    sign = np.where(d < hd // 2, np.float32(-1.0), np.float32(1.0))
    for r in range(R):
        c = bf16_bits_to_f32(cos_t[pos[r]])
        s = bf16_bits_to_f32(sin_t[pos[r]])
        for h in range(H):
            xv = x[r, h]
            if h < nq + nkv:
                t1 = (xv * c).astype(np.float32)
                t2 = ((sign * xv[partner]).astype(np.float32) * s).astype(np.float32)
                o = f32_to_bf16_bits((t1 + t2).astype(np.float32))
            else:
                o = f32_to_bf16_bits(xv)
            if h < nq:
                qo[r, h] = o
            elif h < nq + nkv:
                kc[slot[r], h - nq, pos[r] % ring] = o
            else:
                vc[slot[r], h - nq - nkv, pos[r] % ring] = o
    np.savez_compressed(os.path.join(OUT, "store.npz"), nq=nq, nkv=nkv, hd=hd, ring=ring, sentinel=sentinel,
                        qkv=qkv, bias=bias, cos=cos_t, sin=sin_t, pos=pos, slot=slot, rows=rows, S=S,
                        qo=qo, kc=kc, vc=vc)


def softmax_attend(qrow, K, V, scale):
    s = (K @ qrow) * scale
    s = s - s.max()
    p = np.exp(s)
    return (p[:, None] * V).sum(0) / p.sum()


def decode(rng):
    nq, nkv, hd = 14, 2, 64
    group = nq // nkv
    rows, S = 3, 160
    lens = np.array([1, 77, 160, 129, 64], np.int32)
    rowmap = np.array([2, 0, 1, 1, 0], np.int32)
    b = len(lens)
    q = rand_bf16(rng, (b, nq, hd))
    kc = rand_bf16(rng, (rows, nkv, S, hd))
    vc = rand_bf16(rng, (rows, nkv, S, hd))
    qf = bf16_bits_to_f32(q).astype(np.float64)
    kf = bf16_bits_to_f32(kc).astype(np.float64)
    vf = bf16_bits_to_f32(vc).astype(np.float64)
    scale = hd ** -0.5
    out = np.zeros((b, nq, hd))
    for i in range(b):
        for h in range(nq):
            kh = h // group
            L = lens[i]
            out[i, h] = softmax_attend(qf[i, h], kf[rowmap[i], kh, :L], vf[rowmap[i], kh, :L], scale)
    np.savez_compressed(os.path.join(OUT, "decode.npz"), nq=nq, nkv=nkv, hd=hd, q=q, kc=kc, vc=vc, lens=lens,
                        rowmap=rowmap, out=out.astype(np.float32))


def prefill(rng):
    nq, nkv, hd = 14, 2, 64
    group = nq // nkv
    rows, S = 3, 136
    # requests: (slot, prefix length p0, new tokens n) packed in this order; the last spans two blocks
    reqs = [(1, 20, 5), (2, 0, 3), (0, 64, 70)]
    R = sum(n for _, _, n in reqs)
    q = rand_bf16(rng, (R, nq, hd))
    kc = rand_bf16(rng, (rows, nkv, S, hd))
    vc = rand_bf16(rng, (rows, nkv, S, hd))
    qf = bf16_bits_to_f32(q).astype(np.float64)
    kf = bf16_bits_to_f32(kc).astype(np.float64)
    vf = bf16_bits_to_f32(vc).astype(np.float64)
    scale = hd ** -0.5
    out = np.zeros((R, nq, hd))
    r0 = 0
    for sl, p0, n in reqs:
        for j in range(n):
            for h in range(nq):
                kh = h // group
                out[r0 + j, h] = softmax_attend(qf[r0 + j, h], kf[sl, kh, :p0 + j + 1], vf[sl, kh, :p0 + j + 1], scale)
        r0 += n
    np.savez_compressed(os.path.join(OUT, "prefill.npz"), nq=nq, nkv=nkv, hd=hd, q=q, kc=kc, vc=vc,
                        reqs=np.array(reqs, np.int32), out=out.astype(np.float16))


if __name__ == "__main__":
    rng = np.random.default_rng(20261201)
    rope(rng)
    store(rng)
    decode(rng)
    prefill(rng)
    for f in sorted(os.listdir(OUT)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(OUT, f)))
