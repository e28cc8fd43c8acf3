"""The engine's attention operators on MI355X: drop-ins for the attention part of the reference's
operator module (serve/fast_kernels.py of lvt1693/audio8-turbo-engine), with the same names,
signatures, argument meaning, tensor layouts and error behaviour.

    bias_rope_store(...)                    fast_kernels.py:179-187   (kernel 139-176)
    DecodeAttention(...) / __call__(...)    fast_kernels.py:256-290   (kernels 193-253)
    DecodeAttention.store_and_attend(...)   bias_rope_store then __call__ (fast_engine.py:127-132), one launch
    PrefillPlan(...)                        fast_kernels.py:335-347
    prefill_attention(...)                  fast_kernels.py:350-358   (kernel 296-332)

Every call validates dtypes, devices and strides on the host, then enqueues hand-written gfx950 HIP
kernels on torch's current stream through the C ABI of liba8attn.so (include/a8attn.h). Nothing is
allocated or synchronised inside a call, so a sequence of calls can be captured into a HIP graph
(torch.cuda.graph) and replayed. There is no CPU or framework fallback: if the library is missing
or a launch fails, the call raises.
"""
from __future__ import annotations

import ctypes
from types import SimpleNamespace

import torch

from . import _lib

_BF16 = torch.bfloat16
_I32 = torch.int32


def _need(cond: bool, msg: str, exc=ValueError):
    if not cond:
        raise exc(msg)


def _check_bf16(name: str, t: torch.Tensor, dims: int):
    _need(isinstance(t, torch.Tensor), f"{name} must be a tensor", TypeError)
    _need(t.dtype == _BF16, f"{name} must be bfloat16 (got {t.dtype})", TypeError)
    _need(t.dim() == dims, f"{name} must have {dims} dims (got shape {tuple(t.shape)})")
    _need(t.stride(-1) == 1 or t.shape[-1] == 1, f"{name}: the last dim must be contiguous")


def _check_i32(name: str, t: torch.Tensor, n: int):
    _need(isinstance(t, torch.Tensor), f"{name} must be a tensor", TypeError)
    _need(t.dtype == _I32, f"{name} must be int32 (got {t.dtype})", TypeError)
    _need(t.dim() == 1 and t.is_contiguous(), f"{name} must be a contiguous 1-D tensor")
    _need(t.shape[0] >= n, f"{name} has {t.shape[0]} entries, {n} needed")


def _check_device(**tensors):
    """Every tensor on one HIP device (the kernels dereference all of them there)."""
    devs = {t.device for t in tensors.values() if t is not None}
    for name, t in tensors.items():
        _need(t is None or t.is_cuda, f"{name} must be on a HIP device (got {t.device if t is not None else None})")
    _need(len(devs) == 1, f"all tensors must be on one device (got {sorted(map(str, devs))})")


def _check_cache(kc: torch.Tensor, vc: torch.Tensor, nkv: int, hd: int):
    _check_bf16("kc", kc, 4)
    _check_bf16("vc", vc, 4)
    _need(kc.shape == vc.shape, f"kc {tuple(kc.shape)} and vc {tuple(vc.shape)} must have the same shape")
    # the reference kernels address vc with kc's strides (fast_kernels.py:170, 186, 224-225)
    _need(kc.stride() == vc.stride(), f"kc and vc must share strides ({kc.stride()} vs {vc.stride()})")
    _need(kc.shape[1] == nkv and kc.shape[3] == hd,
          f"cache shape {tuple(kc.shape)} does not match [rows, {nkv}, S, {hd}]")


def _check_store(qkv, bias, cos_tab, sin_tab, pos, slot, qo, kc, vc, nq, nkv, hd, ring):
    """The store arguments' dtypes, shapes, strides and devices; returns the row count."""
    R = qkv.shape[0]
    width = (nq + 2 * nkv) * hd
    _check_bf16("qkv", qkv, 2)
    _need(qkv.shape[1] >= width, f"qkv has {qkv.shape[1]} columns, {width} needed")
    if bias is not None:
        _check_bf16("bias", bias, 1)
        _need(bias.shape[0] >= width, f"bias has {bias.shape[0]} entries, {width} needed")
    _check_bf16("cos_tab", cos_tab, 2)
    _check_bf16("sin_tab", sin_tab, 2)
    _need(cos_tab.shape == sin_tab.shape and cos_tab.stride() == sin_tab.stride(),
          "cos_tab and sin_tab must have the same shape and strides")
    _need(cos_tab.shape[1] >= hd, f"RoPE tables have {cos_tab.shape[1]} columns, {hd} needed")
    _check_i32("pos", pos, R)
    _check_i32("slot", slot, R)
    if qo is not None:
        _check_bf16("qo", qo, 3)
        _need(qo.shape[0] >= R and qo.shape[1] == nq and qo.shape[2] == hd,
              f"qo shape {tuple(qo.shape)} does not match [{R}, {nq}, {hd}]")
    _check_cache(kc, vc, nkv, hd)
    _need(isinstance(ring, int) and 1 <= ring < 2 ** 31, f"ring must be an int in [1, 2^31) (got {ring})")
    _check_device(qkv=qkv, bias=bias, cos_tab=cos_tab, sin_tab=sin_tab, pos=pos, slot=slot, qo=qo, kc=kc, vc=vc)
    return R


def bias_rope_store(qkv, bias, cos_tab, sin_tab, pos, slot, qo, kc, vc, nq, nkv, hd, ring=1 << 30):
    """qkv: [R, (nq+2nkv)*hd]; bias: [(nq+2nkv)*hd] or None. Writes rotated q to qo [R, nq, hd] and k / v
    into kc / vc [Bslots, nkv, S, hd] at [slot, :, pos % ring] (fast_kernels.py:179-187). qo=None: k / v only
    (for prefill_attention_qkv, which forms q from qkv itself).

    Per row r, head h: x = f32(qkv) + f32(bias); q / k get rotate_half RoPE from the bf16 cos / sin tables
    in fp32 and are rounded once to bf16; v is rounded from x. Rows whose position is outside the tables, or
    whose slot / position is outside the cache, store nothing (the reference leaves that undefined)."""
    R = _check_store(qkv, bias, cos_tab, sin_tab, pos, slot, qo, kc, vc, nq, nkv, hd, ring)
    if R == 0:
        return qo
    lib = _lib.load()
    st = lib.a8_bias_rope_store(
        qkv.data_ptr(), qkv.stride(0), bias.data_ptr() if bias is not None else None,
        cos_tab.data_ptr(), sin_tab.data_ptr(), cos_tab.stride(0), cos_tab.shape[0],
        pos.data_ptr(), slot.data_ptr(), R,
        qo.data_ptr() if qo is not None else None, qo.stride(0) if qo is not None else 0,
        qo.stride(1) if qo is not None else 0,
        kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2), kc.shape[0], kc.shape[2],
        nq, nkv, hd, ring, _lib.stream_of(qkv))
    _lib.check(st, "bias_rope_store")
    return qo


def _next_pow2(x: int) -> int:
    return 1 << max(0, (int(x) - 1).bit_length())


class DecodeAttention:
    """Workspace-owning split-K decode attention. The scratch buffers are flat and sized in
    (query row x split) units, so one instance serves both decode (few rows, many splits) and
    packed rows (many rows, one split) with fixed addresses for graph capture
    (fast_kernels.py:256-269).

    Two launch schedules compute the same softmax (split boundaries are not part of the contract):
      mode "split": a8_decode_attn -- the reference's split kernel + combine kernel structure, launch
        shape from a8_decode_choose for this GPU's compute-unit count; the caller's `nsplit` is a lower
        bound on the splits (policy "auto") or exact (policy "caller"). merge_in_kernel = True makes the
        split kernel merge the splits itself (the last split of each (row, kv head) to finish, counters
        in self.counters), so no combine launch follows. Opt-in: measured on MI355X at C2 (64 ragged
        rows, 4 splits) it is slower than the combine launch (15.5 against 15.0 us/layer; the last
        arrival waits for its partial's write-through and the counter's round trip)
      mode "stream": a8_decode_attn_stream -- a persistent kernel that takes fixed-size key chunks in
        turn (whole rows when there are enough of them), plus a small merge kernel for rows longer than
        a chunk; launch shape from a8_decode_choose_stream.
      mode "flat": a8_decode_attn_flat -- one launch for any mix of lengths: the kernel splits the
        rows' actual 64-key tiles evenly over its wavefronts and merges rows spread over several of
        them itself (counters in self.counters); launch shape from a8_decode_choose_flat. Opt-in:
        measured on MI355X it does not beat the others at the engine's shapes (a row merged inside the
        launch pays its memory round trips while the KV stream fills the queues).
      mode "auto" (default): "stream" when the rows are whole units (row, kv head) of 1024+ keys that
        either give every workgroup of the grid two of them -- the peak-load shape -- or, one per
        workgroup, number at least half the compute units (tick buckets of 64-128 slots at KV 2048); for
        the fused store + decode (store_and_attend) also when rows are short (cache_len <= 512: one
        workgroup per (row, kv head) holds the whole row, so the store, the decode and the merge take
        one launch); else "split"."""

    FLAT_MAX_ROWS = 2048

    def __init__(self, cap_row_splits, nq, nkv, hd, nsplit_max, device, scale=None):
        self.nq, self.nkv, self.hd = nq, nkv, hd
        self.group = nq // nkv
        self.gp = max(16, _next_pow2(self.group))
        self.nsplit_max = int(nsplit_max)
        self.cap = int(cap_row_splits)
        self.scale = scale if scale is not None else hd ** -0.5
        self.acc_flat = torch.empty(self.cap * nq * hd, dtype=torch.float32, device=device)
        self.ml_flat = torch.empty(self.cap * nq * 2, dtype=torch.float32, device=device)
        # flat mode and the split mode's in-kernel merge: one arrival counter per (row, kv head); zero
        # between calls (each call re-zeroes what it used)
        self.counters = torch.zeros(self.cap * nkv, dtype=torch.int32, device=device)
        self.merge_in_kernel = False
        dev = torch.device(device)
        self.n_cu = torch.cuda.get_device_properties(dev).multi_processor_count if dev.type == "cuda" else 1
        self.mode = "auto"
        self.policy = "auto"
        self.force_shape = None   # split mode: (nsplit, waves) pins the launch shape (tuning / tests)
        self.force_stream = None  # stream mode: (waves, tiles_per_wave, grid)
        self.force_flat = None    # flat mode: grid
        self._shapes = {}

    def launch_shape(self, b: int, cache_len: int, nsplit: int):
        """Split mode: (key splits, wavefronts per split) for b rows over a cache of cache_len positions."""
        if self.force_shape is not None:
            ns, nw = self.force_shape
            return max(1, min(int(ns), self.cap // max(b, 1))), int(nw)
        key = ("split", b, cache_len, nsplit, self.policy)
        hit = self._shapes.get(key)
        if hit is not None:
            return hit
        ns, nw = ctypes.c_int(0), ctypes.c_int(0)
        nmax = nsplit if self.policy == "caller" else self.nsplit_max
        st = _lib.load().a8_decode_choose(b, self.nkv, cache_len, nsplit, nmax, self.cap, self.n_cu,
                                          ctypes.byref(ns), ctypes.byref(nw))
        _lib.check(st, "decode_choose")
        self._shapes[key] = (ns.value, nw.value)
        return self._shapes[key]

    def stream_shape(self, b: int, cache_len: int):
        """Stream mode: (wavefronts per workgroup, 64-key tiles per wave per chunk, workgroups)."""
        if self.force_stream is not None:
            return tuple(int(x) for x in self.force_stream)
        key = ("stream", b, cache_len)
        hit = self._shapes.get(key)
        if hit is not None:
            return hit
        nw, tpw, grid = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
        st = _lib.load().a8_decode_choose_stream(b, self.nkv, cache_len, self.cap, self.n_cu, ctypes.byref(nw),
                                                 ctypes.byref(tpw), ctypes.byref(grid))
        _lib.check(st, "decode_choose_stream")
        self._shapes[key] = (nw.value, tpw.value, grid.value)
        return self._shapes[key]

    def flat_shape(self, b: int, cache_len: int):
        """Flat mode: (workgroups,)."""
        if self.force_flat is not None:
            return (int(self.force_flat),)
        key = ("flat", b, cache_len)
        hit = self._shapes.get(key)
        if hit is not None:
            return hit
        grid = ctypes.c_int(0)
        st = _lib.load().a8_decode_choose_flat(b, self.nkv, cache_len, self.cap, self.n_cu, ctypes.byref(grid))
        _lib.check(st, "decode_choose_flat")
        self._shapes[key] = (grid.value,)
        return self._shapes[key]

    SHORT_ROWS = 512  # fused calls: rows of at most this many cache positions take one workgroup each

    def short_rows_shape(self, b: int, cache_len: int):
        """Stream mode for short rows: one workgroup per (row, kv head) holding the whole row (up to 4
        waves, the rest in tiles per wave), so no row needs merging across workgroups."""
        tiles = max(1, -(-cache_len // 64))
        nw = 4 if tiles >= 4 else 2 if tiles >= 2 else 1
        return nw, -(-tiles // nw), b * self.nkv

    def schedule(self, b: int, cache_len: int, nsplit: int = 1, fused: bool = False):
        """The schedule a call with b rows over a cache of cache_len positions uses:
        ("stream", (waves, tiles_per_wave, grid)), ("flat", (grid,)) or ("split", (nsplit, waves)).
        fused: the call is a store_and_attend."""
        if self.force_shape is None:
            if self.force_stream is not None or self.mode == "stream":
                return "stream", self.stream_shape(b, cache_len)
            if (self.force_flat is not None or self.mode == "flat") and b <= self.FLAT_MAX_ROWS:
                return "flat", self.flat_shape(b, cache_len)
            if self.mode == "auto":
                if self._stream_pays(b, cache_len):
                    return "stream", self.stream_shape(b, cache_len)
                if fused and 0 < cache_len <= self.SHORT_ROWS:
                    return "stream", self.short_rows_shape(b, cache_len)
        nsplit = max(1, min(int(nsplit), self.nsplit_max))
        return "split", self.launch_shape(b, cache_len, nsplit)

    def _stream_pays(self, b: int, cache_len: int) -> bool:
        """Mode "auto": the streaming schedule for many long rows (see the class docstring)."""
        if cache_len < 1024:
            return False
        nw, tpw, grid = self.stream_shape(b, cache_len)
        whole = nw * tpw * 64 >= cache_len
        units = b * self.nkv
        # two whole units per workgroup, or one per workgroup once the units reach half the compute units
        return whole and (units >= 2 * grid or (grid >= units and 2 * units >= self.n_cu))

    def store_and_attend(self, qkv, bias, cos_tab, sin_tab, pos, slot, q, kc, vc, lens, out, nsplit=1,
                         rowmap=None, ring=1 << 30, phases=3, write_q=True):
        """bias_rope_store(qkv, bias, cos_tab, sin_tab, pos, slot, q, kc, vc, ...) then
        self(q, kc, vc, lens, out, nsplit, rowmap=rowmap): the per-layer pair of fast_engine.py:127-132 with
        the store done by the decode's own kernel (a8_store_decode_stream / _split / _flat, whichever
        schedule the call takes): one launch, or two with the split schedule's combine.
        Same results bit for bit, given that no row attends a cache row another row stores into: the
        engine's decode tick (slot[r] = r, rowmap None, fast_engine.py:752-753) or distinct slots with
        rowmap = slot. Rows sharing a slot, like the fast stack's 2-token first pass, need the two calls.
        The rotated q is an intermediate of the pair that the engine never reads back: with write_q=False
        it is not written (a saving of ~1 us per layer at the peak load). One difference where the
        reference is undefined: a row whose position lies outside the RoPE tables attends with q = 0 here
        (the two calls leave its q row unwritten). A head_dim other than 64 takes the two calls (its kernel
        has no fused store)."""
        if self.hd != 64:
            bias_rope_store(qkv, bias, cos_tab, sin_tab, pos, slot, q, kc, vc, self.nq, self.nkv, self.hd, ring=ring)
            return self(q, kc, vc, lens, out, nsplit, rowmap=rowmap, phases=phases)
        R = _check_store(qkv, bias, cos_tab, sin_tab, pos, slot, q, kc, vc, self.nq, self.nkv, self.hd, ring)
        kind, shape = self.schedule(R, kc.shape[2], nsplit, fused=True)
        _check_i32("lens", lens, R)
        if rowmap is not None:
            _check_i32("rowmap", rowmap, R)
        _check_bf16("out", out, 3)
        _need(out.shape[0] >= R and out.shape[1] == self.nq and out.shape[2] == self.hd,
              f"out shape {tuple(out.shape)} does not match [{R}, {self.nq}, {self.hd}]")
        _check_device(qkv=qkv, kc=kc, lens=lens, rowmap=rowmap, out=out, workspace=self.acc_flat)
        if R == 0:
            return out
        store = (qkv.data_ptr(), qkv.stride(0), bias.data_ptr() if bias is not None else None,
                 cos_tab.data_ptr(), sin_tab.data_ptr(), cos_tab.stride(0), cos_tab.shape[0],
                 pos.data_ptr(), slot.data_ptr(), q.data_ptr() if write_q else None, q.stride(0), q.stride(1),
                 kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2), kc.shape[0], kc.shape[2],
                 lens.data_ptr(), rowmap.data_ptr() if rowmap is not None else None, out.data_ptr(), out.stride(0),
                 out.stride(1), self.acc_flat.data_ptr(), self.ml_flat.data_ptr(), self.cap)
        if kind == "split":
            ns, nw = shape
            st = _lib.load().a8_store_decode_split(*store, *self._split_counters(), R, self.nq, self.nkv, self.hd,
                                                   ring, ns, nw, float(self.scale), int(phases), _lib.stream_of(qkv))
        elif kind == "flat":
            (grid,) = shape
            st = _lib.load().a8_store_decode_flat(*store, self.counters.data_ptr(), self.counters.numel(), R,
                                                  self.nq, self.nkv, self.hd, ring, grid, float(self.scale),
                                                  _lib.stream_of(qkv))
        else:
            nw, tpw, grid = shape
            st = _lib.load().a8_store_decode_stream(*store, R, self.nq, self.nkv, self.hd, ring, nw, tpw, grid,
                                                    float(self.scale), int(phases), _lib.stream_of(qkv))
        _lib.check(st, "store_and_attend")
        return out

    def _split_counters(self):
        """(counters, n_counters) for the split entry points: the in-kernel merge, or (None, 0) for the
        split + combine launches."""
        return (self.counters.data_ptr(), self.counters.numel()) if self.merge_in_kernel else (None, 0)

    def __call__(self, q, kc, vc, lens, out, nsplit=1, bn=64, rowmap=None, phases=3):
        """q: [b, nq, hd]; kc/vc: [rows, nkv, S, hd]; query row i reads cache row rowmap[i]
        (identity when rowmap is None); lens: [b] int32 (keys [0, lens) attended); out: [b, nq, hd]
        (fast_kernels.py:271-290). `phases` (1 = the split / streaming kernel, 2 = the combine / merge
        kernel, 3 = both) lets a profiler time the two kernels apart; callers leave it at 3."""
        b = q.shape[0]
        nsplit = max(1, min(int(nsplit), self.nsplit_max))
        assert b * nsplit <= self.cap, (b, nsplit, self.cap)
        _need(bn == 64, f"bn={bn}: only 64-key tiles are implemented", NotImplementedError)
        if q.dtype == torch.float32:
            return self._call_f32q(q, kc, vc, lens, out, rowmap)
        _need(q.dtype == _BF16, f"q must be bfloat16 or float32 (got {q.dtype})", TypeError)
        _check_bf16("q", q, 3)
        _need(q.shape[1] == self.nq and q.shape[2] == self.hd,
              f"q shape {tuple(q.shape)} does not match [b, {self.nq}, {self.hd}]")
        _check_cache(kc, vc, self.nkv, self.hd)
        _check_i32("lens", lens, b)
        if rowmap is not None:
            _check_i32("rowmap", rowmap, b)
        _check_bf16("out", out, 3)
        _need(out.shape[0] >= b and out.shape[1] == self.nq and out.shape[2] == self.hd,
              f"out shape {tuple(out.shape)} does not match [{b}, {self.nq}, {self.hd}]")
        _check_device(q=q, kc=kc, vc=vc, lens=lens, rowmap=rowmap, out=out, workspace=self.acc_flat)
        if b == 0:
            return out
        lib = _lib.load()
        common = (q.data_ptr(), q.stride(0), q.stride(1),
                  kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2), kc.shape[0], kc.shape[2],
                  lens.data_ptr(), rowmap.data_ptr() if rowmap is not None else None,
                  out.data_ptr(), out.stride(0), out.stride(1), self.acc_flat.data_ptr(), self.ml_flat.data_ptr())
        kind, shape = self.schedule(b, kc.shape[2], nsplit)
        if kind == "flat":
            (grid,) = shape
            st = lib.a8_decode_attn_flat(*common, self.cap, self.counters.data_ptr(), self.counters.numel(), b,
                                         self.nq, self.nkv, self.hd, grid, float(self.scale), _lib.stream_of(q))
            _lib.check(st, "decode_attention")
            return out
        if kind == "stream":
            nw, tpw, grid = shape
            st = lib.a8_decode_attn_stream(*common, self.cap, b, self.nq, self.nkv, self.hd, nw, tpw, grid,
                                           float(self.scale), int(phases), _lib.stream_of(q))
            _lib.check(st, "decode_attention")
            return out
        ns, nw = shape
        st = lib.a8_decode_attn(*common, self.cap, *self._split_counters(), b, self.nq, self.nkv, self.hd, ns, nw,
                                float(self.scale), int(phases), _lib.stream_of(q))
        _lib.check(st, "decode_attention")
        return out


    def _call_f32q(self, q, kc, vc, lens, out, rowmap):
        """fp32 queries: the reference's PREC = "ieee" branch (fast_kernels.py:279; fp32 products, bf16 weights in
        P.V, the output in out's dtype, bf16 or fp32) through a8_decode_attn_f32q, one launch (the engine never
        decodes an fp32 q; the kernel is exact, not tuned)."""
        b = q.shape[0]
        _need(q.dim() == 3 and q.stride(2) == 1 and q.shape[1] == self.nq and q.shape[2] == self.hd,
              f"q shape {tuple(q.shape)} does not match [b, {self.nq}, {self.hd}] with a contiguous last dim")
        _check_cache(kc, vc, self.nkv, self.hd)
        _check_i32("lens", lens, b)
        if rowmap is not None:
            _check_i32("rowmap", rowmap, b)
        _need(isinstance(out, torch.Tensor) and out.dtype in (_BF16, torch.float32) and out.dim() == 3 and
              out.stride(2) == 1, "out must be a bfloat16 or float32 [b, nq, hd] tensor with a contiguous last dim",
              TypeError)
        _need(out.shape[0] >= b and out.shape[1] == self.nq and out.shape[2] == self.hd,
              f"out shape {tuple(out.shape)} does not match [{b}, {self.nq}, {self.hd}]")
        _check_device(q=q, kc=kc, vc=vc, lens=lens, rowmap=rowmap, out=out)
        if b == 0:
            return out
        st = _lib.load().a8_decode_attn_f32q(
            q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
            kc.stride(2), kc.shape[0], kc.shape[2], lens.data_ptr(), rowmap.data_ptr() if rowmap is not None else None,
            out.data_ptr(), out.stride(0), out.stride(1), 1 if out.dtype == torch.float32 else 0, b, self.nq,
            self.nkv, self.hd, float(self.scale), _lib.stream_of(q))
        _lib.check(st, "decode_attention (fp32 q)")
        return out

def heaviest_first(blocks):
    """(q0, n, slot, pos0) query blocks sorted by their key count pos0 + n, largest first; stable."""
    return sorted(blocks, key=lambda b: -(b[3] + b[1]))


class PrefillPlan:
    """Query-block schedule for a packed prefill: request i's rows [r0_i, r0_i+n_i) sit at
    positions [p0_i, p0_i+n_i) of cache row slot_i (keys [0, p0_i) are an already-stored prefix)
    (fast_kernels.py:335-347). q0, n, slot, pos0 are the reference's blocks in its order (request order).
    `dispatch` holds the same blocks heaviest first (most keys, ties in request order): the kernel
    dispatches its workgroups in that list's order, so the long blocks start first and the short ones fill
    the end. Every block writes its own rows, so the order changes no result."""
    BM = 64

    def __init__(self, r0s, ns, slots, p0s, device):
        blocks = [(r0 + off, min(self.BM, n - off), s, p0 + off)
                  for r0, n, s, p0 in zip(r0s, ns, slots, p0s) for off in range(0, n, self.BM)]
        cols = [list(c) for c in zip(*blocks)] if blocks else [[], [], [], []]
        dcols = [list(c) for c in zip(*heaviest_first(blocks))] if blocks else [[], [], [], []]
        t = torch.tensor(cols + dcols, dtype=torch.int32)
        if torch.device(device).type == "cuda":
            t = t.pin_memory().to(device, non_blocking=True)
        self.q0, self.n, self.slot, self.pos0 = t[0], t[1], t[2], t[3]
        self.dispatch = SimpleNamespace(q0=t[4], n=t[5], slot=t[6], pos0=t[7])
        self.nblk = len(blocks)


def prefill_attention(q, kc, vc, plan, out, group, scale=None):
    """q/out: [R, nq, hd] packed rows; kc/vc: [rows, nkv, S, hd] (fast_kernels.py:350-358).
    `plan` is a PrefillPlan or any object with int32 device tensors q0, n, slot, pos0, an int nblk and
    BM = 64 (the graph-mode plan of fast_engine.py:825-826). When the plan carries `dispatch` (the same
    blocks in the order to launch them: PrefillPlan, PrefillMeta.plan), the kernel reads that list."""
    _check_bf16("q", q, 3)
    nq, hd = q.shape[1], q.shape[2]
    scale = scale if scale is not None else hd ** -0.5
    _need(group >= 1 and nq % group == 0, f"group {group} does not divide nq {nq}")
    _check_cache(kc, vc, nq // group, hd)
    _check_bf16("out", out, 3)
    _need(out.shape[0] >= q.shape[0] and out.shape[1:] == q.shape[1:],
          f"out shape {tuple(out.shape)} does not match q {tuple(q.shape)}")
    bm = int(getattr(plan, "BM", PrefillPlan.BM))
    nblk = int(plan.nblk)
    blocks = getattr(plan, "dispatch", None) or plan
    for name in ("q0", "n", "slot", "pos0"):
        _check_i32(f"plan.{name}", getattr(blocks, name), nblk)
    _check_device(q=q, kc=kc, vc=vc, out=out, **{f"plan.{k}": getattr(blocks, k) for k in ("q0", "n", "slot", "pos0")})
    if nblk == 0 or q.shape[0] == 0:
        return out
    st = _lib.load().a8_prefill_attn(
        q.data_ptr(), q.stride(0), q.stride(1), q.shape[0],
        kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2), kc.shape[0], kc.shape[2],
        out.data_ptr(), out.stride(0), out.stride(1),
        blocks.q0.data_ptr(), blocks.n.data_ptr(), blocks.slot.data_ptr(), blocks.pos0.data_ptr(), nblk, bm,
        nq, group, hd, float(scale), _lib.stream_of(q))
    _lib.check(st, "prefill_attention")
    return out


def prefill_attention_qkv(qkv, bias, cos_tab, sin_tab, kc, vc, plan, out, group, scale=None):
    """prefill_attention with q formed from the qkv rows inside the launch (a8_prefill_attn_qkv): the q that
    bias_rope_store(qkv, bias, cos_tab, sin_tab, pos, ...) would write, at each row's position = its block's
    pos0 + the row's index in the block, with the store's arithmetic -- so, after
    bias_rope_store(..., qo=None, ...), the two calls leave the same out bits as bias_rope_store then
    prefill_attention, without writing or re-reading q. No counterpart in the reference (fast_engine.py:127-132
    makes the two calls). qkv [R, (nq+2nkv)*hd]; out [R, nq, hd]; head_dim 64; other arguments as
    prefill_attention. A query at a position outside the tables attends with q = 0."""
    _check_bf16("qkv", qkv, 2)
    _check_bf16("out", out, 3)
    nq, hd = out.shape[1], out.shape[2]
    _need(group >= 1 and nq % group == 0, f"group {group} does not divide nq {nq}")
    nkv = nq // group
    width = (nq + 2 * nkv) * hd
    _need(qkv.shape[1] >= width, f"qkv has {qkv.shape[1]} columns, {width} needed")
    _need(out.shape[0] >= qkv.shape[0], f"out has {out.shape[0]} rows, qkv {qkv.shape[0]}")
    if bias is not None:
        _check_bf16("bias", bias, 1)
        _need(bias.shape[0] >= width, f"bias has {bias.shape[0]} entries, {width} needed")
    _check_bf16("cos_tab", cos_tab, 2)
    _check_bf16("sin_tab", sin_tab, 2)
    _need(cos_tab.shape == sin_tab.shape and cos_tab.stride() == sin_tab.stride(),
          "cos_tab and sin_tab must have the same shape and strides")
    _need(cos_tab.shape[1] >= hd, f"RoPE tables have {cos_tab.shape[1]} columns, {hd} needed")
    scale = scale if scale is not None else hd ** -0.5
    _check_cache(kc, vc, nkv, hd)
    bm = int(getattr(plan, "BM", PrefillPlan.BM))
    nblk = int(plan.nblk)
    blocks = getattr(plan, "dispatch", None) or plan
    for name in ("q0", "n", "slot", "pos0"):
        _check_i32(f"plan.{name}", getattr(blocks, name), nblk)
    _check_device(qkv=qkv, bias=bias, cos_tab=cos_tab, sin_tab=sin_tab, kc=kc, vc=vc, out=out,
                  **{f"plan.{k}": getattr(blocks, k) for k in ("q0", "n", "slot", "pos0")})
    if nblk == 0 or qkv.shape[0] == 0:
        return out
    st = _lib.load().a8_prefill_attn_qkv(
        qkv.data_ptr(), qkv.stride(0), bias.data_ptr() if bias is not None else None,
        cos_tab.data_ptr(), sin_tab.data_ptr(), cos_tab.stride(0), cos_tab.shape[0], qkv.shape[0],
        kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2), kc.shape[0], kc.shape[2],
        out.data_ptr(), out.stride(0), out.stride(1),
        blocks.q0.data_ptr(), blocks.n.data_ptr(), blocks.slot.data_ptr(), blocks.pos0.data_ptr(), nblk, bm,
        nq, group, hd, float(scale), _lib.stream_of(qkv))
    _lib.check(st, "prefill_attention_qkv")
    return out


def prefix_copy(k, v, kc_all, vc_all, slots):
    """kc_all[:, slots, :, :Lp] = k.unsqueeze(1) and vc_all[:, slots, :, :Lp] = v.unsqueeze(1) in one launch:
    a voice prefix's K/V ([layers, nkv, Lp, hd] each, from _prefix_kv) into the cache rows of the requests
    that use it (fast_engine.py:1098-1103; caches [layers, rows, nkv, S, hd]). `slots` is an int32 tensor on
    the device (or a list, uploaded here). A slot outside the cache is skipped (the reference's index-put
    would raise)."""
    _check_bf16("k", k, 4)
    _check_bf16("v", v, 4)
    _need(k.shape == v.shape and k.stride() == v.stride(), "k and v must have the same shape and strides")
    _check_bf16("kc_all", kc_all, 5)
    _check_bf16("vc_all", vc_all, 5)
    _need(kc_all.shape == vc_all.shape and kc_all.stride() == vc_all.stride(),
          "kc_all and vc_all must have the same shape and strides")
    layers, nkv, Lp, hd = k.shape
    _need(kc_all.shape[0] == layers and kc_all.shape[2] == nkv and kc_all.shape[4] == hd,
          f"cache shape {tuple(kc_all.shape)} does not match [{layers}, rows, {nkv}, S, {hd}]")
    _need(Lp <= kc_all.shape[3], f"prefix of {Lp} positions does not fit a cache of {kc_all.shape[3]}")
    if not isinstance(slots, torch.Tensor):
        slots = torch.tensor(list(slots), dtype=_I32)
        if kc_all.is_cuda:
            slots = slots.pin_memory().to(kc_all.device, non_blocking=True)
    _check_i32("slots", slots, 0)
    _check_device(k=k, v=v, kc_all=kc_all, vc_all=vc_all, slots=slots)
    n = slots.shape[0]
    if n == 0 or layers == 0 or Lp == 0:
        return
    st = _lib.load().a8_prefix_copy(
        k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        kc_all.data_ptr(), vc_all.data_ptr(), kc_all.stride(0), kc_all.stride(1), kc_all.stride(2), kc_all.stride(3),
        slots.data_ptr(), n, layers, nkv, Lp, hd, kc_all.shape[1], kc_all.shape[3], _lib.stream_of(kc_all))
    _lib.check(st, "prefix_copy")


def rmsnorm(x, w, eps, residual=None, out=None, res_out=None):
    """x: [..., N] bf16. With residual: h = x + residual (bf16, stored to res_out, default in place into
    residual) and returns (rmsnorm(h), h); without: returns rmsnorm(x) (fast_kernels.py:49-69, kernel 30-46:
    fp32 sum of squares, xn rounded to bf16, then weight * xn rounded to bf16)."""
    _need(isinstance(x, torch.Tensor) and x.dtype == _BF16, "x must be a bfloat16 tensor", TypeError)
    N = x.shape[-1]
    x2 = x.reshape(-1, N)
    y = out if out is not None else torch.empty_like(x)
    y2 = y.reshape(-1, N)
    _check_bf16("w", w, 1)
    _need(w.shape[0] == N, f"w has {w.shape[0]} entries, {N} needed")
    for name, t in (("x", x2), ("out", y2)):
        _need(t.stride(-1) == 1, f"{name}: the last dim must be contiguous")
    r2 = ro2 = None
    if residual is not None:
        _need(residual.dtype == _BF16 and residual.shape[-1] == N, "residual must be bfloat16 of the same width")
        ro = res_out if res_out is not None else residual
        r2, ro2 = residual.reshape(-1, N), ro.reshape(-1, N)
        _need(r2.shape[0] == x2.shape[0] and ro2.shape[0] == x2.shape[0], "residual rows must match x")
        _need(r2.stride(-1) == 1 and ro2.stride(-1) == 1, "residual: the last dim must be contiguous")
    _check_device(x=x2, w=w, out=y2, residual=r2, res_out=ro2)
    st = _lib.load().a8_rmsnorm(x2.data_ptr(), x2.stride(0), r2.data_ptr() if r2 is not None else None,
                                r2.stride(0) if r2 is not None else 0, w.data_ptr(), y2.data_ptr(), y2.stride(0),
                                ro2.data_ptr() if ro2 is not None else None, ro2.stride(0) if ro2 is not None else 0,
                                x2.shape[0], N, float(eps), _lib.stream_of(x2))
    _lib.check(st, "rmsnorm")
    return (y, ro) if residual is not None else y


def silu_mul(gu, out=None):
    """gu: [..., 2I] bf16 -> [..., I]: bf16(bf16(silu(g)) * u) with g, u the two halves
    (fast_kernels.py:537-545, kernel 526-534)."""
    _need(isinstance(gu, torch.Tensor) and gu.dtype == _BF16, "gu must be a bfloat16 tensor", TypeError)
    I = gu.shape[-1] // 2
    g2 = gu.reshape(-1, 2 * I)
    y = out if out is not None else torch.empty(*gu.shape[:-1], I, dtype=gu.dtype, device=gu.device)
    y2 = y.reshape(-1, I)
    _need(g2.stride(-1) == 1 and y2.stride(-1) == 1, "gu / out: the last dim must be contiguous")
    _check_device(gu=g2, out=y2)
    st = _lib.load().a8_silu_mul(g2.data_ptr(), g2.stride(0), y2.data_ptr(), y2.stride(0), g2.shape[0], I,
                                 _lib.stream_of(g2))
    _lib.check(st, "silu_mul")
    return y


def gemm_ws_bytes(M, N, splits):
    """Workspace bytes gemm_small needs for `splits` k ranges (0 for one): 4096 bytes of tile counters, then
    the fp32 partials. Allocate it zeroed (torch.zeros): every call leaves the counters at zero."""
    return 0 if splits <= 1 else 4096 + splits * M * N * 4


def gemm_small(x, w, out=None, splits=1, ws=None, mblocks=1):
    """out[M, N] = x[M, K] @ w[N, K]^T with this package's small-M kernel (a8_gemm_small): bf16, fp32
    accumulation, M <= 192, K a multiple of 64, N of 8. splits > 1 splits K across workgroups, with fp32
    partials in `ws` (a device tensor of at least gemm_ws_bytes(M, N, splits) bytes, zeroed when allocated)
    summed in a fixed order by each tile's last workgroup;
    mblocks > 1 splits the token rows into blocks (more workgroups for narrow N). Neither changes the result.
    Raises (A8Error) where the kernel does not apply; GemmDispatch only calls it where it does."""
    _check_bf16("x", x, 2)
    _check_bf16("w", w, 2)
    M, K = x.shape
    N = w.shape[0]
    _need(w.shape[1] == K, f"w shape {tuple(w.shape)} does not match K = {K}")
    y = out if out is not None else torch.empty(M, N, dtype=x.dtype, device=x.device)
    _check_bf16("out", y, 2)
    _need(y.shape[0] == M and y.shape[1] == N, f"out shape {tuple(y.shape)} does not match [{M}, {N}]")
    _check_device(x=x, w=w, out=y, ws=ws)
    st = _lib.load().a8_gemm_small(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), y.data_ptr(), y.stride(0),
                                   ws.data_ptr() if ws is not None else None,
                                   ws.numel() * ws.element_size() if ws is not None else 0, M, N, K, int(splits),
                                   int(mblocks), _lib.stream_of(x))
    _lib.check(st, "gemm_small")
    return y


def gemm_silu_small(x, w13, out=None, mblocks=1):
    """out[M, I] = silu_mul(x @ w13^T) in one launch (a8_gemm_silu_small): w13 [2I, K] = [gate; up] rows, the
    product rounded to bf16 as gemm_small's output, then silu_mul's arithmetic (fast_kernels.py:526-545) in the
    GEMM's epilogue: the same bits as silu_mul(gemm_small(x, w13)). M <= 192, K a multiple of 64, I of 8."""
    _check_bf16("x", x, 2)
    _check_bf16("w13", w13, 2)
    M, K = x.shape
    _need(w13.shape[1] == K and w13.shape[0] % 2 == 0, f"w13 shape {tuple(w13.shape)} must be [2I, {K}]")
    I = w13.shape[0] // 2
    y = out if out is not None else torch.empty(M, I, dtype=x.dtype, device=x.device)
    _check_bf16("out", y, 2)
    _need(y.shape[0] == M and y.shape[1] == I, f"out shape {tuple(y.shape)} does not match [{M}, {I}]")
    _check_device(x=x, w13=w13, out=y)
    st = _lib.load().a8_gemm_silu_small(x.data_ptr(), x.stride(0), w13.data_ptr(), w13.stride(0), y.data_ptr(),
                                        y.stride(0), M, I, K, int(mblocks), _lib.stream_of(x))
    _lib.check(st, "gemm_silu_small")
    return y


def gemm_small_norm(x, w, out, splits=1, mblocks=1, ws=None, gated=False, res_add=False, ss_out=None, ss_in=None,
                    eps=1e-6, prefetch=None, pf_sink=None, pf_slices=8):
    """The slow-AR projections with the residual RMSNorm between them folded in (a8_gemm_small_norm; the
    reference runs rmsnorm, fast_kernels.py:30-69, as its own launch between the products):
      res_add: out is the residual stream, updated in place: out = bf16(bf16(x @ w^T) + out) -- the product
        rounded to bf16 and rmsnorm's residual add, the same bits; ss_out (fp32 [M, N / 32], optional) gets the
        new stream's sums of squares per 32-column group, the next norm's statistic;
      ss_in: x is a raw residual stream h and w a weight with the norm's weight folded in (fold_norm): out =
        bf16((h @ w^T) * rsqrt(sum(ss_in[m]) / K + eps)) -- the norm's 1 / rms applied to the fp32 products
        (the reference rounds h * (1 / rms) and its product with the norm weight to bf16 first: within bf16
        rounding noise of it); with gated, w = [gate; up] and out = silu_mul of the two (gemm_silu_small's
        epilogue).
    M <= 192, K a multiple of 64, N of 8 (32 with ss_out, 16 gated); splits / ws / mblocks as gemm_small.
    prefetch (a contiguous device tensor, with pf_sink: 16 device bytes): pf_slices more grid slices of
    workgroups read it once while the product runs (a8_gemm_small_norm_pf: the next product's weights into the
    memory-side cache); the result is the same."""
    _check_bf16("x", x, 2)
    _check_bf16("w", w, 2)
    M, K = x.shape
    N = w.shape[0]
    _need(w.shape[1] == K, f"w shape {tuple(w.shape)} does not match K = {K}")
    _check_bf16("out", out, 2)
    _need(out.shape[0] == M and out.shape[1] == (N // 2 if gated else N), f"out shape {tuple(out.shape)} mismatch")
    for name, t in (("ss_out", ss_out), ("ss_in", ss_in)):
        if t is not None:
            _need(t.dtype == torch.float32 and t.dim() == 2 and t.is_contiguous() and t.shape[0] >= M,
                  f"{name} must be a contiguous float32 [>= M, groups] tensor")
    if ss_out is not None:
        _need(ss_out.shape[1] == N // 32, f"ss_out must have N / 32 = {N // 32} columns")
    _check_device(x=x, w=w, out=out, ws=ws, ss_out=ss_out, ss_in=ss_in, prefetch=prefetch, pf_sink=pf_sink)
    args = [x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), out.data_ptr(), out.stride(0),
            ws.data_ptr() if ws is not None else None, ws.numel() * ws.element_size() if ws is not None else 0,
            M, N, K, int(splits), int(mblocks), int(bool(gated)), int(bool(res_add)),
            ss_out.data_ptr() if ss_out is not None else None, ss_in.data_ptr() if ss_in is not None else None,
            ss_in.shape[1] if ss_in is not None else 0, float(eps)]
    if prefetch is not None:
        _need(prefetch.is_contiguous() and pf_sink is not None and pf_sink.numel() * pf_sink.element_size() >= 16,
              "prefetch must be contiguous, with a 16-byte pf_sink")
        st = _lib.load().a8_gemm_small_norm_pf(*args, prefetch.data_ptr(), prefetch.numel() * prefetch.element_size(),
                                               pf_sink.data_ptr(), int(pf_slices), _lib.stream_of(x))
    else:
        st = _lib.load().a8_gemm_small_norm(*args, _lib.stream_of(x))
    _lib.check(st, "gemm_small_norm")
    return out


def fold_norm(w, norm_w):
    """w [N, K] with the norm weight [K] folded in, for gemm_small_norm(ss_in=...): bf16(w * norm_w)."""
    return (w.float() * norm_w.float()[None, :]).to(w.dtype).contiguous()


class GemmDispatch:
    """Per-(M, N, K) choice between the library GEMM (torch.matmul -> hipBLASLt) and gemm_small, measured on
    the running GPU at startup, outside graph capture (the reference's GemmDispatch, fast_kernels.py:413-519,
    chooses between cuBLAS and tuned Triton configs the same way). `tune(weights, Ms)` times both (with each
    split count) for every weight shape and token count; `__call__(x, w)` then takes the faster, and the
    library GEMM for shapes not tuned. The split partials share one workspace sized by tune (calls on one
    instance run in stream order). Prefill-sized M (over 192 rows) always takes the library GEMM: tune records
    its time at `large_m` rows per shape. With `cache_path`, results persist in a JSON file keyed by GPU, so
    a later startup times only what the file lacks."""

    SPLITS = (1, 2, 3, 4, 7, 8, 14)
    MBLOCKS = (1, 2, 3, 6)

    def __init__(self):
        self.small = {}     # (M, N, K) -> (splits, mblocks) or None (library GEMM)
        self.small_best = {}  # (M, N, K) -> the fastest gemm_small (splits, mblocks), chosen or not
        self.gated_best = {}  # (M, N, K) -> the fastest gemm_silu_small (1, mblocks) for the gated weights
        self.large = {}     # (N, K) -> the prefill-sized record: {"M", "choice": "library", "us", "TFLOP/s"}
        self.enabled = True
        self.ws = None
        self.log = []

    @staticmethod
    def _time(fns, n=20, reps=7):
        """Time of one call, from a graph of n calls cycling through `fns` (one per weight of the shape, so that
        with a model's layers the weights are not all served from cache): the median over `reps` timed replays
        (one timed replay pair left the choice between shapes within ~1 us of each other to noise)."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for f in fns[:2]:
                f()
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                fns[i % len(fns)]()
        g.replay()
        g.replay()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        ev[0].record()
        for i in range(reps):
            g.replay()
            ev[i + 1].record()
        torch.cuda.synchronize()
        ts = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(reps))
        return ts[reps // 2] / n

    @staticmethod
    def applies(M, N, K):
        return 0 < M <= 192 and K % 64 == 0 and N % 8 == 0

    @staticmethod
    def gpu_key(device) -> str:
        """The tuning cache's key for a GPU: architecture, compute units and name (the name alone can be empty
        or generic on ROCm)."""
        p = torch.cuda.get_device_properties(device)
        return f"{getattr(p, 'gcnArchName', '?')}/{p.multi_processor_count}CU/{p.name}"

    def _cache_load(self, cache_path, gpu):
        import json
        import os
        if not cache_path or not os.path.exists(cache_path):
            return {}
        try:
            with open(cache_path) as f:
                return json.load(f).get(gpu, {})
        except (OSError, ValueError):
            return {}

    def _cache_store(self, cache_path, gpu, entries):
        import json
        import os
        try:
            with open(cache_path) as f:
                allc = json.load(f)
        except (OSError, ValueError):
            allc = {}
        allc.setdefault(gpu, {}).update(entries)
        tmp = f"{cache_path}.{os.getpid()}.tmp"
        with open(tmp, "w") as f:
            json.dump(allc, f, indent=1, sort_keys=True)
        os.replace(tmp, cache_path)

    @torch.inference_mode()
    def tune(self, weights, Ms, log=None, gated=(), large_m=4096, cache_path=None):
        """weights: iterable of [N, K] bf16 tensors (a model's projections: the calls are timed cycling through
        every weight of a shape, as the model's layers would); Ms: token counts. gated: those of the weights that
        are [gate; up] products (w13): their shape is also timed through the launch that runs it with the
        activation in its epilogue (gemm_silu_small), whose best row-block count `gated` and the norm-fused
        products then take.
        large_m: the prefill-sized token count each weight shape is also timed at (M > 192, where only the
        library GEMM applies: the choice recorded in `large` is the library, with its time).
        cache_path: a JSON file of results keyed by GPU (gpu_key), as the reference keeps its tuning
        (fast_kernels.py:442-505): shapes found there are not timed again, new results are merged into it."""
        shapes = {}
        for w in weights:
            shapes.setdefault((w.shape[0], w.shape[1]), []).append(w)
        gshapes = {}
        for w in gated:
            gshapes.setdefault((w.shape[0], w.shape[1]), []).append(w)
        if not shapes:
            return
        dev = next(iter(shapes.values()))[0].device
        gpu = self.gpu_key(dev)
        disk = self._cache_load(cache_path, gpu)
        fresh = {}
        need = 0

        def tup(v):
            return None if v is None else tuple(int(a) for a in v)

        for (N, K), ws_ in shapes.items():
            for M in sorted(set(int(m) for m in Ms)):
                key = f"{M},{N},{K}"
                gkey = (N, K) in gshapes and N % 16 == 0
                if not self.applies(M, N, K):
                    self.small[(M, N, K)] = None
                    continue
                if f"s{key}" in disk and (not gkey or f"g{key}" in disk):
                    self.small[(M, N, K)] = tup(disk[f"s{key}"])
                    if disk.get(f"b{key}") is not None:
                        self.small_best[(M, N, K)] = tup(disk[f"b{key}"])
                    if gkey and disk.get(f"g{key}") is not None:
                        self.gated_best[(M, N, K)] = tup(disk[f"g{key}"])
                    lib_us, best_us = disk.get(f"t{key}", [None, None])
                    self.log.append(((M, N, K), None if lib_us is None else lib_us / 1e3, self.small[(M, N, K)],
                                     None if best_us is None else best_us / 1e3))
                else:
                    x = torch.randn(M, K, device=dev, dtype=ws_[0].dtype)
                    y = torch.empty(M, N, device=dev, dtype=ws_[0].dtype)
                    n = max(20, len(ws_))
                    best, best_t = None, self._time([lambda w=w: torch.matmul(x, w.t(), out=y) for w in ws_], n)
                    lib_t = best_t
                    small_t = None
                    for sp in self.SPLITS:
                        if sp > K // 64:
                            continue
                        wsp = torch.zeros(gemm_ws_bytes(M, N, sp), dtype=torch.uint8, device=dev) if sp > 1 else None
                        for mb in self.MBLOCKS:
                            if mb > 1 and (M + mb - 1) // mb < 32:
                                continue
                            t = self._time([lambda w=w: gemm_small(x, w, y, splits=sp, ws=wsp, mblocks=mb)
                                            for w in ws_], n)
                            if t < best_t:
                                best, best_t = (sp, mb), t
                            if small_t is None or t < small_t:
                                self.small_best[(M, N, K)], small_t = (sp, mb), t
                    self.small[(M, N, K)] = best
                    if gkey:
                        gws = gshapes[(N, K)]
                        yg = torch.empty(M, N // 2, device=dev, dtype=x.dtype)
                        gt = None
                        for mb in self.MBLOCKS:
                            if mb > 1 and (M + mb - 1) // mb < 32:
                                continue
                            t = self._time([lambda w=w: gemm_silu_small(x, w, yg, mblocks=mb) for w in gws],
                                           max(20, len(gws)))
                            if gt is None or t < gt:
                                self.gated_best[(M, N, K)], gt = (1, mb), t
                    self.log.append(((M, N, K), lib_t, best, best_t))
                    fresh[f"s{key}"] = None if best is None else list(best)
                    fresh[f"b{key}"] = None if (M, N, K) not in self.small_best else list(self.small_best[(M, N, K)])
                    if gkey:
                        fresh[f"g{key}"] = (None if (M, N, K) not in self.gated_best
                                            else list(self.gated_best[(M, N, K)]))
                    fresh[f"t{key}"] = [round(lib_t * 1e3, 3), round(best_t * 1e3, 3)]
                    if log:
                        log(f"[gemm] M={M} N={N} K={K}: library {lib_t * 1e3:.1f} us, "
                            + (f"gemm_small splits={best[0]} mblocks={best[1]} {best_t * 1e3:.1f} us" if best
                               else "kept"))
                sb = self.small_best.get((M, N, K))
                if sb is not None and sb[0] > 1:  # the norm-fused products run gemm_small whatever was chosen
                    need = max(need, gemm_ws_bytes(M, N, sb[0]))
            # prefill-sized M: the library GEMM (gemm_small serves M <= 192); its time is recorded
            if large_m and int(large_m) > 192:
                lkey = f"l{N},{K}"
                if lkey in disk:
                    self.large[(N, K)] = disk[lkey]
                else:
                    M = int(large_m)
                    x = torch.randn(M, K, device=dev, dtype=ws_[0].dtype)
                    y = torch.empty(M, N, device=dev, dtype=ws_[0].dtype)
                    t = self._time([lambda w=w: torch.matmul(x, w.t(), out=y) for w in ws_], 5, reps=3)
                    ent = {"M": M, "choice": "library", "us": round(t * 1e3, 2),
                           "TFLOP/s": round(2 * M * N * K / t / 1e9, 1)}
                    self.large[(N, K)] = ent
                    fresh[lkey] = ent
                    del x, y
        if need and (self.ws is None or self.ws.numel() < need):
            self.ws = torch.zeros(need, dtype=torch.uint8, device=dev)  # the tile counters start at zero
        if cache_path and fresh:
            self._cache_store(cache_path, gpu, fresh)
        if log and cache_path:
            log(f"[gemm] {len(fresh)} entries timed, the rest from {cache_path}")

    @staticmethod
    def _operands_ok(x, w):
        """gemm_small's operand layout: 2-D, unit column strides, 16-byte aligned rows (pointers and row
        strides); anything else takes torch.matmul, as the reference's mm would."""
        return (x.dim() == 2 and w.dim() == 2 and x.stride(1) == 1 and w.stride(1) == 1
                and x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0 and x.stride(0) % 8 == 0 and w.stride(0) % 8 == 0)

    def __call__(self, x, w):
        if not self.enabled or not self._operands_ok(x, w):
            return torch.matmul(x, w.t())
        best = self.small.get((x.shape[0], w.shape[0], w.shape[1]))
        if best is None:
            return torch.matmul(x, w.t())
        sp, mb = best
        return gemm_small(x, w, splits=sp, ws=self.ws if sp > 1 else None, mblocks=mb)

    def gated(self, x, w13):
        """silu_mul(self(x, w13)): where the tuned choice for w13 is gemm_small in one pass (no k splits), the
        activation runs in its epilogue (gemm_silu_small, same bits, one launch and no [M, 2I] round trip);
        otherwise the product, then silu_mul."""
        key = (x.shape[0], w13.shape[0], w13.shape[1])
        best = self.small.get(key) if self.enabled and self._operands_ok(x, w13) else None
        if best is not None and best[0] == 1:
            return gemm_silu_small(x, w13, mblocks=self.gated_best.get(key, best)[1])
        return silu_mul(self(x, w13))

    def _shape(self, M, N, K, gated):
        """(splits, mblocks) of gemm_small for a norm-fused product (which only gemm_small computes): the
        fastest gemm_small shape tune measured (gated: the fastest gated launch, where tune timed one), else one
        pass over K with row blocks of about 32 rows for narrow N; gated: one pass."""
        if gated and (M, N, K) in self.gated_best:
            return self.gated_best[(M, N, K)]
        best = self.small_best.get((M, N, K))
        if best is not None and (not gated or best[0] == 1):
            return best
        return 1, (1 if N >= 4096 else max(1, M // 32))

    def residual(self, x, w, res, ss_out=None, prefetch=None, pf_sink=None, pf_slices=8):
        """res += x @ w^T in place (the product rounded to bf16, then the residual add: rmsnorm's residual
        step), with the new stream's per-row sums of squares into ss_out ([M, N / 32] fp32); prefetch / pf_sink
        as gemm_small_norm's."""
        sp, mb = self._shape(x.shape[0], w.shape[0], w.shape[1], False)
        return gemm_small_norm(x, w, res, splits=sp, mblocks=mb, ws=self.ws if sp > 1 else None, res_add=True,
                               ss_out=ss_out, prefetch=prefetch, pf_sink=pf_sink, pf_slices=pf_slices)

    def normed(self, h, wf, ss_in, eps, out, gated=False, prefetch=None, pf_sink=None, pf_slices=8):
        """The product of RMSNorm(h) with a weight whose norm weight is folded in (fold_norm), the norm's
        statistic from the producer's ss_out; gated: silu_mul of the [gate; up] halves."""
        sp, mb = self._shape(h.shape[0], wf.shape[0], wf.shape[1], gated)
        return gemm_small_norm(h, wf, out, splits=sp, mblocks=mb, ws=self.ws if sp > 1 else None, gated=gated,
                               ss_in=ss_in, eps=eps, prefetch=prefetch, pf_sink=pf_sink, pf_slices=pf_slices)


_F16 = torch.float16


def conv_cl(xin, w, bias, TR, taps, dil, ph, out, res=None, f16acc=True, cfg=None, snake=None, ws=None):
    """Channels-last causal / transposed conv as an implicit GEMM (fast_kernels.py:600-623, kernel 551-597):
    xin [B, Tin, Cin] fp16; w [ph, taps, Cin, Cout_pad] fp16 with Cout_pad a multiple of 8 (its rows are read
    16 bytes at a time; the reference pads to max(16, Cout)); out [B, TR*ph, >=Cout] with Cout =
    out.shape[-1], any view: out[b, t*ph + p] = bias + sum_j xin[b, t + j*dil] @ w[p, j] (+ res[b, t*ph + p]).
    snake = (alpha, 1/(alpha+eps)) fp32 [Cin] applies x + ib sin(alpha x)^2 to xin on the load. Accumulation
    is fp32 (f16acc, the reference's fp16 slice sums, and cfg, its Triton tile choice, are accepted and
    unused). ws: an optional device byte buffer the launch may use to split K on short inputs (its size:
    conv_cl_ws_bytes); without one, or when it is too small, K is not split. Nothing is allocated here."""
    for name, t, d in (("xin", xin, 3), ("w", w, 4), ("out", out, 3)):
        _need(isinstance(t, torch.Tensor) and t.dtype == _F16, f"{name} must be a float16 tensor", TypeError)
        _need(t.dim() == d and t.stride(-1) == 1, f"{name} must have {d} dims with a contiguous last dim")
    B, Tin, Cin = xin.shape
    Cout = out.shape[-1]
    _need(w.shape[0] == ph and w.shape[1] == taps and w.shape[2] == Cin and w.shape[3] >= Cout,
          f"w {tuple(w.shape)} does not match [{ph}, {taps}, {Cin}, >={Cout}]")
    _need(out.shape[0] == B and out.shape[1] >= TR * ph, f"out {tuple(out.shape)} does not hold [{B}, {TR * ph}, ...]")
    if bias is not None:
        _need(bias.dtype == _F16 and bias.dim() == 1 and bias.shape[0] >= Cout and bias.is_contiguous(),
              "bias must be a contiguous float16 vector of >= Cout entries")
    if res is not None:
        _need(res.dtype == _F16 and res.dim() == 3 and res.stride(-1) == 1 and res.shape[0] == B and
              res.shape[1] >= TR * ph and res.shape[2] >= Cout, "res must be float16 like out")
    sa = sib = None
    if snake is not None:
        sa, sib = snake
        _need(sa.dtype == torch.float32 and sib.dtype == torch.float32 and sa.is_contiguous() and sib.is_contiguous()
              and sa.numel() >= Cin and sib.numel() >= Cin, "snake must be two contiguous float32 [Cin] vectors")
    _check_device(xin=xin, w=w, out=out, bias=bias, res=res, snake_a=sa, snake_ib=sib)
    if ws is not None:
        _need(isinstance(ws, torch.Tensor) and ws.is_contiguous() and ws.device == xin.device,
              "ws must be a contiguous device tensor on xin's device")
    lib = _lib.load()
    st = lib.a8_conv_cl(
        xin.data_ptr(), xin.stride(0), xin.stride(1), w.data_ptr(), w.stride(0), w.stride(1), w.stride(2),
        w.shape[3], bias.data_ptr() if bias is not None else None, res.data_ptr() if res is not None else None,
        res.stride(0) if res is not None else 0, res.stride(1) if res is not None else 0, out.data_ptr(),
        out.stride(0), out.stride(1), sa.data_ptr() if sa is not None else None,
        sib.data_ptr() if sib is not None else None, B, Tin, TR, Cin, Cout, taps, dil, ph,
        ws.data_ptr() if ws is not None else None, ws.numel() * ws.element_size() if ws is not None else 0,
        _lib.stream_of(xin))
    _lib.check(st, "conv_cl")
    return out


def ru_cl(xin, w1, b1, a2, ib2, w2, b2, res, out, TR, taps, dil):
    """One whole residual unit in one launch (the reference's ru_fused, fast_kernels.py:626-692):
        out[b, t] = res[b, t] + b2 + snake2(bias1 + sum_j xin[b, t + j*dil] @ w1[j]) @ w2
    with xin [B, Tin, C] the activated input ([state | snake1(x)], snake_cat's output), w1 [taps, C, C] and w2
    [C, C] fp16 ([k][n], CLConv's packing without the phase dim), b1 / b2 fp16 [C], a2 / ib2 the second snake's
    fp32 [C] vectors, res the unit's raw input [B, >=TR, C]. The first conv's output h stays in registers in
    fp32 (h + b1, the snake, one rounding to fp16), as in ru_fused; accumulation is fp32 throughout. C is 96,
    192 or 384 (one workgroup tile holds a row's channels)."""
    for name, t, d in (("xin", xin, 3), ("w1", w1, 3), ("w2", w2, 2), ("res", res, 3), ("out", out, 3)):
        _need(isinstance(t, torch.Tensor) and t.dtype == _F16, f"{name} must be a float16 tensor", TypeError)
        _need(t.dim() == d and t.stride(-1) == 1, f"{name} must have {d} dims with a contiguous last dim")
    B, Tin, C = xin.shape
    _need(w1.shape == (taps, C, C) and w1.stride(1) == C, f"w1 {tuple(w1.shape)} must be [{taps}, {C}, {C}], rows of {C}")
    _need(w2.shape == (C, C) and w2.stride(0) == C, f"w2 {tuple(w2.shape)} must be [{C}, {C}], contiguous")
    _need(res.shape[0] == B and res.shape[1] >= TR and res.shape[2] == C, f"res {tuple(res.shape)} must be [{B}, >={TR}, {C}]")
    _need(out.shape[0] == B and out.shape[1] >= TR and out.shape[2] == C, f"out {tuple(out.shape)} must be [{B}, >={TR}, {C}]")
    for name, v, dt in (("b1", b1, _F16), ("b2", b2, _F16), ("a2", a2, torch.float32), ("ib2", ib2, torch.float32)):
        _need(isinstance(v, torch.Tensor) and v.dtype == dt and v.is_contiguous() and v.numel() >= C,
              f"{name} must be a contiguous {dt} vector of >= {C} entries")
    _check_device(xin=xin, w1=w1, w2=w2, res=res, out=out, b1=b1, b2=b2, a2=a2, ib2=ib2)
    st = _lib.load().a8_ru_cl(
        xin.data_ptr(), xin.stride(0), xin.stride(1), w1.data_ptr(), w1.stride(0), w1.stride(1), b1.data_ptr(),
        a2.data_ptr(), ib2.data_ptr(), w2.data_ptr(), b2.data_ptr(), res.data_ptr(), res.stride(0), res.stride(1),
        out.data_ptr(), out.stride(0), out.stride(1), B, Tin, TR, C, taps, dil, _lib.stream_of(xin))
    _lib.check(st, "ru_cl")
    return out


def conv_cl_ws_bytes(B, TR, Cin, Cout, taps, ph):
    """Bytes of the split-K workspace conv_cl uses for this shape (0: K is not split)."""
    return int(_lib.load().a8_conv_cl_ws_bytes(B, TR, Cin, Cout, taps, ph))


def conv_out_tanh(x, state, a, ib, w, bias, out):
    """The decoder's last conv with what surrounds it, in one launch (a8_conv_out_tanh): out[b, t] =
    tanh(fp16(bias + sum_j [state | snake(x)][b, t + j] . w[j])) in fp32, and state <- the last CTX rows of
    [state | snake(x)] (serve/fast_engine.py:228-233 and 310: snake_cat, conv_cl into one channel, the state
    refresh, y[..., 0].float().tanh()). x [B, T, Cin] raw fp16; state [>=B, CTX, Cin] activated, CTX = taps - 1
    <= T; a / ib fp32 [Cin]; w [taps, Cin] fp16 (the one output channel); bias fp16 [1] or None; out [B, T] fp32
    (row stride free). Cin a multiple of 8 up to 128, taps up to 8."""
    _need(isinstance(x, torch.Tensor) and x.dim() == 3 and x.stride(-1) == 1 and x.dtype == _F16,
          "x must be float16 [B, T, Cin], last dim contiguous")
    B, T, Cin = x.shape
    taps = w.shape[0]
    _need(w.dtype == _F16 and w.dim() == 2 and w.shape[1] == Cin and w.is_contiguous(), "w must be float16 [taps, Cin]")
    _need(state is not None and state.dtype == _F16 and state.shape[0] >= B and state.shape[1] == taps - 1 and
          state.shape[2] == Cin and state.stride(-1) == 1, "state must be float16 [>=B, taps - 1, Cin]")
    _need(out.dtype == torch.float32 and out.dim() == 2 and out.shape[0] == B and out.shape[1] == T and
          out.stride(-1) == 1, "out must be float32 [B, T]")
    _need(a.dtype == torch.float32 and ib.dtype == torch.float32 and a.is_contiguous() and ib.is_contiguous()
          and a.numel() >= Cin and ib.numel() >= Cin, f"a / ib must be contiguous float32 vectors of >= {Cin}")
    _need(bias is None or (bias.dtype == _F16 and bias.numel() >= 1), "bias must be None or float16 [1]")
    _check_device(x=x, state=state, w=w, out=out, a=a, ib=ib, bias=bias)
    st = _lib.load().a8_conv_out_tanh(
        x.data_ptr(), x.stride(0), x.stride(1), state.data_ptr(), state.stride(0), state.stride(1), a.data_ptr(),
        ib.data_ptr(), w.data_ptr(), bias.data_ptr() if bias is not None else None, out.data_ptr(), out.stride(0),
        B, T, state.shape[1], Cin, taps, _lib.stream_of(x))
    _lib.check(st, "conv_out_tanh")
    return out


def snake_cat(x, state, a, ib, out, refresh=False):
    """x [B, T, C] (raw) and state [>=B, CTX, C] (activated context, or None) -> out [B, CTX+T, C] =
    concat(state, snake(x)) along time (fast_kernels.py:718-729, kernel 695-715); a / ib None: no snake.
    refresh=True (T >= CTX) also writes the next context into state, state[:B] = out[:, T:], in the same
    launch (a8_snake_cat_refresh; the reference copies it after the conv, fast_engine.py:232)."""
    _need(isinstance(x, torch.Tensor) and x.dim() == 3 and x.stride(-1) == 1, "x must be [B, T, C], last dim contiguous")
    B, T, C = x.shape
    CTX = state.shape[1] if state is not None else 0
    _need(out.dim() == 3 and out.shape[0] == B and out.shape[1] >= CTX + T and out.shape[2] == C and
          out.stride(-1) == 1 and out.dtype == x.dtype, "out must be [B, CTX+T, C] like x")
    if state is not None:
        _need(state.dtype == x.dtype and state.shape[0] >= B and state.shape[2] == C and state.stride(-1) == 1,
              "state must be [>=B, CTX, C] like x")
    if a is not None:
        _need(a.dtype == torch.float32 and ib.dtype == torch.float32 and a.is_contiguous() and ib.is_contiguous()
              and a.numel() >= C and ib.numel() >= C, "a / ib must be contiguous float32 [C] vectors")
    _need(x.dtype == _F16, "x must be float16", TypeError)
    _check_device(x=x, state=state, out=out, a=a, ib=ib)
    if refresh:
        _need(state is not None and T >= CTX, "refresh needs a state and T >= CTX")
    fn = _lib.load().a8_snake_cat_refresh if refresh else _lib.load().a8_snake_cat
    st = fn(
        x.data_ptr(), x.stride(0), x.stride(1), state.data_ptr() if state is not None else None,
        state.stride(0) if state is not None else 0, state.stride(1) if state is not None else 0,
        a.data_ptr() if a is not None else None, ib.data_ptr() if ib is not None else None, out.data_ptr(),
        out.stride(0), out.stride(1), B, T, CTX, C, _lib.stream_of(out))
    _lib.check(st, "snake_cat")
    return out
