"""The attention slice of the reference's transformer stack and its caller-side plumbing
(serve/fast_engine.py of lvt1693/audio8-turbo-engine):

    rope_tables(base, hd, n, dev)          fast_engine.py:70-75   (_rope_tables)
    permute_qk(w, nq, nkv, hd)             fast_engine.py:60-67   (_permute_qk)
    ref_nsplit(b, nkv)                     fast_engine.py:776     (the reference's per-bucket split count)
    AttnStack                              fast_engine.py:82-138  (_Stack: KV-cache layout + per-layer order)
    PrefillMeta                            fast_engine.py:681-691, 820-853 (graph-mode prefill plan buffer)

AttnStack keeps the reference's KV-cache contract -- kc_all / vc_all [layers, rows, nkv, S, hd] bf16 with
kc[i] / vc[i] the per-layer views -- and its per-layer call order (bias_rope_store, then decode or packed
prefill attention). The projections, norms and MLP between layers are outside this path: a caller hands
each layer's fused qkv rows in.
"""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import torch

from .fast_kernels import (DecodeAttention, PrefillPlan, bias_rope_store, heaviest_first, prefill_attention,
                           prefill_attention_qkv)


def rope_tables(base, hd, n, dev):
    """cos / sin [n, hd] bf16 for rotate_half: fp32 phases pos * base^(-2i/hd) rounded to bf16 and
    duplicated to [c, c] / [s, s] (fast_engine.py:70-75). Computed on the host in fp32 and uploaded, so
    every device sees the same table."""
    fr = 1.0 / (base ** (torch.arange(0, hd, 2).float()[: hd // 2] / hd))
    ph = torch.outer(torch.arange(n).float(), fr)
    c, s = ph.cos().to(torch.bfloat16), ph.sin().to(torch.bfloat16)
    return torch.cat([c, c], -1).contiguous().to(dev), torch.cat([s, s], -1).contiguous().to(dev)


def permute_qk(w, nq, nkv, hd):
    """Rows of a fused [q | k | v] projection (weight [N, K] or bias [N]) with every q / k head's dims
    reordered from interleaved RoPE pairs (2i, 2i+1) to rotate_half halves (i, i + hd/2); v rows unchanged
    (fast_engine.py:60-67). q . k is unchanged by the reorder."""
    p = torch.cat([torch.arange(0, hd, 2), torch.arange(1, hd, 2)]).to(w.device)
    rest = w.shape[1:]
    q = w[:nq * hd].reshape(nq, hd, *rest)[:, p].reshape(nq * hd, *rest)
    k = w[nq * hd:(nq + nkv) * hd].reshape(nkv, hd, *rest)[:, p].reshape(nkv * hd, *rest)
    return torch.cat([q, k, w[(nq + nkv) * hd:]], 0).contiguous()


def ref_nsplit(b, nkv):
    """The reference's split count per tick bucket, tuned for an 84-SM GPU (fast_engine.py:776):
    max(1, min(16, ceil(168 / (b * nkv)))). DecodeAttention takes it as a lower bound."""
    return max(1, min(16, -(-2 * 84 // (b * nkv))))


class AttnStack:
    """KV caches + attention of an n-layer stack (the attention part of fast_engine.py:82-138).

    forward(qkv, bias, pos, slot, lens, ...) processes R token rows: row r is at RoPE position pos[r],
    its K/V goes into cache row slot[r] at column pos[r] % ring, and it attends columns [0, lens[r]) of
    that cache row (decode), or its request's causal range (packed prefill, when a plan is given)."""

    def __init__(self, n_layers, nq, nkv, hd, rope_base, max_rows, cache_rows, cache_len, max_pos, dev,
                 dt=torch.bfloat16, nsplit_max=16, ring=None):
        self.nq, self.nkv, self.hd = nq, nkv, hd
        self.n_layers = n_layers
        self.cos, self.sin = rope_tables(rope_base, hd, max_pos, dev)
        self.ring = int(ring) if ring else 1 << 30
        self.kc_all = torch.zeros(n_layers, cache_rows, nkv, cache_len, hd, dtype=dt, device=dev)
        self.vc_all = torch.zeros_like(self.kc_all)
        self.kc = list(self.kc_all.unbind(0))
        self.vc = list(self.vc_all.unbind(0))
        self.attn = DecodeAttention(max_rows, nq, nkv, hd, nsplit_max, dev)

    def layer(self, i, qkv, bias, pos, slot, lens, q, o, nsplit=1, rowmap=True, plan=None, fuse=False):
        """Layer i's attention (fast_engine.py:127-132): store, then attend. q / o: [R, nq, hd] buffers.

        fuse=True declares that no row attends a cache row that another row of the call stores into (the
        slow stack's decode tick: slot[r] = r with rowmap off, fast_engine.py:752-753; or distinct slots
        with rowmap on); the decode then stores and attends in one launch where the schedule allows
        (DecodeAttention.store_and_attend), with the same results. Rows sharing a slot (the fast stack's
        2-token pass) must keep fuse=False. With a plan (the admission's packed prefill), fuse=True stores
        k / v only and the prefill forms q from qkv itself (prefill_attention_qkv; each row's position is its
        block's pos0 + its index in the block, as the plan of an admission has it): the same out bits, and q
        is neither written nor read (head_dim 64; at 128 it makes the two calls)."""
        if plan is None and fuse:
            return self.attn.store_and_attend(qkv, bias, self.cos, self.sin, pos, slot, q, self.kc[i], self.vc[i],
                                              lens, o, nsplit=nsplit, rowmap=slot if rowmap else None,
                                              ring=self.ring, write_q=False)
        if plan is not None and fuse and self.hd == 64:
            bias_rope_store(qkv, bias, self.cos, self.sin, pos, slot, None, self.kc[i], self.vc[i],
                            self.nq, self.nkv, self.hd, ring=self.ring)
            return prefill_attention_qkv(qkv, bias, self.cos, self.sin, self.kc[i], self.vc[i], plan, o,
                                         self.nq // self.nkv)
        bias_rope_store(qkv, bias, self.cos, self.sin, pos, slot, q, self.kc[i], self.vc[i],
                        self.nq, self.nkv, self.hd, ring=self.ring)
        if plan is not None:
            prefill_attention(q, self.kc[i], self.vc[i], plan, o, self.nq // self.nkv)
        else:
            self.attn(q, self.kc[i], self.vc[i], lens, o, nsplit=nsplit, rowmap=slot if rowmap else None)
        return o

    def forward(self, qkv, bias, pos, slot, lens, nsplit=1, rowmap=True, plan=None, q=None, outs=None, fuse=False):
        """All layers in order. qkv / bias: per-layer lists ([R, (nq+2nkv)*hd] rows, [(nq+2nkv)*hd] or None).
        outs: per-layer [R, nq, hd] outputs (allocated when None; pass buffers under graph capture)."""
        R = qkv[0].shape[0]
        dev = qkv[0].device
        if q is None:
            q = torch.empty(R, self.nq, self.hd, dtype=torch.bfloat16, device=dev)
        if outs is None:
            outs = [torch.empty(R, self.nq, self.hd, dtype=torch.bfloat16, device=dev) for _ in range(self.n_layers)]
        for i in range(self.n_layers):
            self.layer(i, qkv[i], bias[i] if bias is not None else None, pos, slot, lens, q, outs[i],
                       nsplit=nsplit, rowmap=rowmap, plan=plan, fuse=fuse)
        return outs


class PrefillMeta:
    """The graph-mode packed-prefill plan: one int32 device buffer
    [pos NT | slot NT | q0, n, bslot, pos0 NB | last, st, cpos NR | dq0, dn, dbslot, dpos0 NB] with
    NB = NT/64 + NR, rewritten by one host-to-device copy per admission and read by a captured prefill
    (fast_engine.py:681-691, 820-853). The first nine fields are the reference's layout and contents; the
    last four hold the same blocks heaviest first, the order the kernel dispatches them in (see
    PrefillPlan). Padding rows, blocks and requests point at the scratch cache row `scr` with n = 0 and
    pos = 0."""

    FIELDS = ("pos", "slot", "q0", "n", "bslot", "pos0", "last", "st", "cpos", "dq0", "dn", "dbslot", "dpos0")

    def __init__(self, NT, NR, scr, dev):
        BM = PrefillPlan.BM
        self.NT, self.NR, self.NB, self.scr = NT, NR, NT // BM + NR, scr
        NB = self.NB
        self.off = np.cumsum([0, NT, NT, NB, NB, NB, NB, NR, NR, NR, NB, NB, NB, NB])
        self.buf = torch.zeros(int(self.off[-1]), dtype=torch.int32, device=dev)
        self.v = SimpleNamespace(**{k: self.buf[self.off[i]:self.off[i + 1]] for i, k in enumerate(self.FIELDS)})

    def host(self, nt, slots, ns, starts):
        """Host int32 contents for requests of ns tokens at positions starts.. in slots, packed in order
        (fast_engine.py:837-853); the dispatch copy of the query blocks is heaviest first."""
        BM, o = PrefillPlan.BM, self.off
        m = np.zeros(int(o[-1]), np.int32)
        pos, slot, q0, n, bslot, p0, last, st, cpos, dq0, dn, dbslot, dp0 = (m[o[i]:o[i + 1]] for i in range(13))
        slot[:], bslot[:], st[:], dbslot[:] = self.scr, self.scr, self.scr, self.scr
        r0, blocks = 0, []
        for k, (s, cnt, a) in enumerate(zip(slots, ns, starts)):
            pos[r0:r0 + cnt] = np.arange(a, a + cnt)
            slot[r0:r0 + cnt] = s
            blocks += [(r0 + off, min(BM, cnt - off), s, a + off) for off in range(0, cnt, BM)]
            last[k], st[k], cpos[k] = r0 + cnt - 1, s, a + cnt
            r0 += cnt
        bi = len(blocks)
        assert r0 <= nt and bi <= nt // BM + self.NR and len(slots) <= self.NR
        if bi:
            q0[:bi], n[:bi], bslot[:bi], p0[:bi] = zip(*blocks)
            dq0[:bi], dn[:bi], dbslot[:bi], dp0[:bi] = zip(*heaviest_first(blocks))
        return m

    def load(self, nt, slots, ns, starts):
        """Write the plan for one admission into the device buffer (one pinned host-to-device copy)."""
        h = torch.from_numpy(self.host(nt, slots, ns, starts))
        if self.buf.is_cuda:
            h = h.pin_memory()
        self.buf.copy_(h, non_blocking=True)

    def plan(self, nt):
        """The duck-typed block plan a captured prefill of nt tokens passes to prefill_attention
        (fast_engine.py:824-826): nt/64 + NR blocks, padding blocks are no-ops."""
        v, nb = self.v, nt // PrefillPlan.BM + self.NR
        return SimpleNamespace(q0=v.q0[:nb], n=v.n[:nb], slot=v.bslot[:nb], pos0=v.pos0[:nb], nblk=nb,
                               BM=PrefillPlan.BM,
                               dispatch=SimpleNamespace(q0=v.dq0[:nb], n=v.dn[:nb], slot=v.dbslot[:nb],
                                                        pos0=v.dpos0[:nb]))
