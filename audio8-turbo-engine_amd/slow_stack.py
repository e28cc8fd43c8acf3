"""The slow AR's transformer stack around the attention path (reference serve/fast_engine.py:82-138, _Stack).

Per layer (fast_engine.py:117-138): qkv = h @ wqkv^T -> bias + RoPE + K/V store -> decode (or packed prefill)
attention -> a = o @ wo^T -> (h, res) = rmsnorm(a, ln2, residual=res) -> m = silu_mul(h @ w13^T) @ w2^T ->
(h, res) = rmsnorm(m, next ln1 or the final norm, residual=res). The attention is AttnStack (this package's
kernels, the reference's cache layout and store-then-attend order); the norms and the gated activation are
this package's kernels (rmsnorm, silu_mul); the four projections go through `mm`, the reference's argument
(fast_engine.py:90): torch.matmul (hipBLASLt) by default, or a GemmDispatch, which takes this package's
small-M GEMM (gemm_small) for the shapes where it measured faster.

Weights are the reference's fused layout per layer: wqkv [(nq+2nkv)hd, hidden] (q/k rows already in
rotate_half order, fast_engine.py:100-101), bqkv or None, wo [hidden, nq hd], w13 = cat(w1, w3) [2 inter,
hidden], w2 [hidden, inter], ln1 / ln2 [hidden], and the final norm. Without a checkpoint (none exists
offline) `random_weights` draws a synthetic set of that shape."""
from __future__ import annotations

import torch

from .attn_stack import AttnStack
from .fast_kernels import GemmDispatch, fold_norm, rmsnorm, silu_mul


def random_weights(n_layers, hidden, nq, nkv, hd, inter, dev, seed=0, dt=torch.bfloat16):
    """Synthetic weights of the slow AR's shapes: projections ~ N(0, 1/fan_in) (unit-variance outputs),
    biases ~ N(0, 0.02^2), norm weights ~ 1 + N(0, 0.05^2)."""
    g = torch.Generator(device=dev).manual_seed(seed)

    def lin(n, k):
        return (torch.randn(n, k, generator=g, device=dev) / k ** 0.5).to(dt)

    def vec(n, mean, std):
        return (mean + std * torch.randn(n, generator=g, device=dev)).to(dt)

    W = (nq + 2 * nkv) * hd
    layers = [dict(wqkv=lin(W, hidden), bqkv=vec(W, 0.0, 0.02), wo=lin(hidden, nq * hd), w13=lin(2 * inter, hidden),
                   w2=lin(hidden, inter), ln1=vec(hidden, 1.0, 0.05), ln2=vec(hidden, 1.0, 0.05))
              for _ in range(n_layers)]
    return layers, vec(hidden, 1.0, 0.05)


class SlowStack:
    """forward(x, pos, slot, lens, nsplit=1, rowmap=True, plan=None) as _Stack.forward (fast_engine.py:117-138):
    R independent token rows, row r at RoPE position pos[r], its K/V stored into cache row slot[r] and
    attending columns [0, lens[r]) of cache row slot[r] (rowmap) or r; with a PrefillPlan the packed causal
    prefill instead. Returns the final-normed hidden [R, hidden]; `x` is consumed (the residual stream is
    updated in place), as in the reference. fuse=True lets the store and the decode share one launch where
    every row attends its own slot (AttnStack.forward)."""

    # token rows up to which a norm-fused step applies (gemm_small_norm's M limit)
    FUSE_NORM_ROWS = 192

    def __init__(self, layers, norm, nq, nkv, hd, eps, rope_base, max_rows, cache_rows, cache_len, max_pos, dev,
                 nsplit_max=16, ring=None, mm=None):
        self.layers = layers
        self.norm = norm
        self.nq, self.nkv, self.hd, self.eps = nq, nkv, hd, float(eps)
        self.attn = AttnStack(len(layers), nq, nkv, hd, rope_base, max_rows, cache_rows, cache_len, max_pos, dev,
                              nsplit_max=nsplit_max, ring=ring)
        self.kc_all, self.vc_all = self.attn.kc_all, self.attn.vc_all
        self.kc, self.vc = self.attn.kc, self.attn.vc
        # the projections' GEMM: the reference's `mm` argument (fast_engine.py:90) -- torch.matmul by default, or
        # a GemmDispatch (this package's small-M kernel where it measured faster)
        self.mm = mm if mm is not None else (lambda x, w: torch.matmul(x, w.t()))
        # fuse_norm: with a GemmDispatch as mm, decode steps of at most FUSE_NORM_ROWS rows run the residual
        # RMSNorms inside the projections (gemm_small_norm): the o / w2 products add the residual in their epilogue
        # and leave the next norm's sums of squares; the qkv / w13 products take that norm's 1 / rms on their fp32
        # products, its weight folded into theirs -- two launches fewer per layer, within bf16 rounding noise of
        # the reference's rmsnorm -> product sequence
        self.fuse_norm = False
        self._folded = None  # built on the first norm-fused step and kept (refold() rebuilds it)
        self._shapes_ok = None
        self._ss = None
        # prefetch_w13 (norm-fused steps): the o projection's launch carries extra workgroups that read the layer's
        # w13 weights once (gemm_small_norm prefetch), so the w13 product finds them in the memory-side cache
        self.prefetch_w13 = True
        self.pf_slices = 8  # grid slices of prefetch workgroups (each as many as the o product's weight tiles)
        # prefetch_kv_bytes: the qkv product's launch (layers after the first) also reads about this many bytes of
        # the layer's K cache -- the last rows of the tick, which the whole-row decode reaches in its second pass --
        # into the memory-side cache, at most a sixth of the rows. Off: since the decode streams K and V by
        # non-temporal DMA it gains nothing from it (192 rows x 2048, one box: 0 / 8 / 16 / 24 MB -> 69.85 /
        # 70.17 / 70.53 / 70.49 us per layer; with the register-loaded K it had saved 0.55 us).
        self.prefetch_kv_bytes = 0
        self.kv_slices = 8
        self._sink = None

    def _fused_shapes_ok(self):
        """The shapes gemm_small_norm serves: the residual stream's sums of squares in hidden / 32 groups, at
        most 32 and a multiple of 4, every product's K a multiple of 64, the gated w13 a multiple of 16 rows.
        Other models take the unfused path."""
        hidden = self.norm.shape[0]
        if hidden % 32 or not (4 <= hidden // 32 <= 32) or (hidden // 32) % 4:
            return False
        for L in self.layers:
            for name in ("wqkv", "wo", "w13", "w2"):
                if L[name].shape[1] % 64:
                    return False
            if L["w13"].shape[0] % 16:
                return False
        return True

    def refold(self):
        """Rebuilds the norm-folded weights (fold_norm of wqkv / w13 with their norm weights) the norm-fused steps
        use. They are built on the first such step and kept: call this after changing any layer's wqkv, w13, ln1
        or ln2 in place."""
        self._folded = None

    def _fused_ready(self, R, plan):
        if not (self.fuse_norm and isinstance(self.mm, GemmDispatch) and plan is None and R <= self.FUSE_NORM_ROWS):
            return False
        if self._shapes_ok is None:
            self._shapes_ok = self._fused_shapes_ok()
        if not self._shapes_ok:
            return False
        hidden = self.norm.shape[0]
        if self._folded is None:
            self._folded = [(fold_norm(L["wqkv"], L["ln1"]), fold_norm(L["w13"], L["ln2"])) for L in self.layers]
            dev = self.norm.device
            self._ss = [torch.zeros(self.FUSE_NORM_ROWS, hidden // 32, dtype=torch.float32, device=dev) for _ in range(2)]
            self._sink = torch.zeros(4, dtype=torch.int32, device=dev)
        return True

    def _forward_fused(self, x, pos, slot, lens, nsplit, rowmap, fuse):
        """forward() with the residual RMSNorms inside the projections (see fuse_norm)."""
        R = x.shape[0]
        mm = self.mm
        h = rmsnorm(x, self.layers[0]["ln1"], self.eps)
        res = x
        q = torch.empty(R, self.nq, self.hd, dtype=x.dtype, device=x.device)
        o = torch.empty_like(q)
        ss_a, ss_b = self._ss[0][:R], self._ss[1][:R]
        for i, L in enumerate(self.layers):
            wqkv_f, w13_f = self._folded[i]
            if i == 0:
                qkv = mm(h, L["wqkv"])
            else:  # RMSNorm(res, ln1) folded in, its statistic from the previous layer's w2 product
                pk = None
                row_bytes = self.kc[i][0].numel() * self.kc[i].element_size()
                n = min(R // 6, self.prefetch_kv_bytes // row_bytes) if self.prefetch_w13 else 0
                if n > 0 and self.kc[i].is_contiguous():
                    r0 = max(0, min(R, self.kc[i].shape[0]) - n)
                    pk = self.kc[i][r0:r0 + n]
                qkv = mm.normed(res, wqkv_f, ss_b, self.eps, torch.empty(R, wqkv_f.shape[0], dtype=x.dtype,
                                                                          device=x.device),
                                prefetch=pk, pf_sink=self._sink, pf_slices=self.kv_slices)
            self.attn.layer(i, qkv, L["bqkv"], pos, slot, lens, q, o, nsplit=nsplit, rowmap=rowmap, fuse=fuse)
            mm.residual(o.view(R, -1), L["wo"], res, ss_a,          # res += o @ wo^T
                        prefetch=w13_f if self.prefetch_w13 else None, pf_sink=self._sink, pf_slices=self.pf_slices)
            act = mm.normed(res, w13_f, ss_a, self.eps, torch.empty(R, w13_f.shape[0] // 2, dtype=x.dtype,
                                                                    device=x.device), gated=True)
            mm.residual(act, L["w2"], res, ss_b)                    # res += act @ w2^T
        return rmsnorm(res, self.norm, self.eps)

    def forward(self, x, pos, slot, lens, nsplit=1, rowmap=True, plan=None, fuse=False):
        R = x.shape[0]
        if self._fused_ready(R, plan):
            return self._forward_fused(x, pos, slot, lens, nsplit, rowmap, fuse)
        nl = len(self.layers)
        h = rmsnorm(x, self.layers[0]["ln1"], self.eps)
        res = x
        q = torch.empty(R, self.nq, self.hd, dtype=x.dtype, device=x.device)
        o = torch.empty_like(q)
        for i, L in enumerate(self.layers):
            qkv = self.mm(h, L["wqkv"])
            self.attn.layer(i, qkv, L["bqkv"], pos, slot, lens, q, o, nsplit=nsplit, rowmap=rowmap, plan=plan,
                            fuse=fuse)
            a = self.mm(o.view(R, -1), L["wo"])
            h, res = rmsnorm(a, L["ln2"], self.eps, residual=res)
            # a GemmDispatch runs the activation in the w13 product's epilogue where it takes gemm_small
            act = self.mm.gated(h, L["w13"]) if hasattr(self.mm, "gated") else silu_mul(self.mm(h, L["w13"]))
            m = self.mm(act, L["w2"])
            nxt = self.layers[i + 1]["ln1"] if i + 1 < nl else self.norm
            h, res = rmsnorm(m, nxt, self.eps, residual=res)
        return h
