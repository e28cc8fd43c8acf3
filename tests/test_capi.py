"""The C-ABI library on the host (no GPU needed): it loads, exports every symbol include/a8attn.h declares,
rejects bad arguments before launching anything, and its launch-shape policy keeps its contract."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "a8attn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(a8_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    assert set(declared_functions()) == {"a8_version", "a8_last_error", "a8_hip_runtime_path", "a8_bias_rope_store",
                                         "a8_decode_attn", "a8_decode_attn_noalloc", "a8_decode_choose", "a8_decode_attn_stream",
                                         "a8_decode_choose_stream", "a8_store_decode_stream", "a8_prefill_attn", "a8_prefill_attn_qkv",
                                         "a8_decode_attn_flat", "a8_decode_choose_flat", "a8_store_decode_flat",
                                         "a8_store_decode_split", "a8_prefix_copy", "a8_rmsnorm", "a8_silu_mul", "a8_gemm_small", "a8_gemm_silu_small", "a8_gemm_small_norm", "a8_ru_cl", "a8_decode_attn_f32q",
                                         "a8_conv_cl", "a8_conv_cl_ws_bytes", "a8_snake_cat", "a8_conv_out_tanh", "a8_snake_cat_refresh", "a8_gemm_small_norm_pf"}


def test_library_is_built_from_these_sources(a8):
    """The library in the tree carries the hash of the sources it was built from: a build older than an edit
    to csrc/ or include/ fails here (rebuild with `python __graft_entry__.py build`)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("_a8_bl", os.path.join(ROOT, "audio8-turbo-engine_amd", "build_lib.py"))
    bl = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bl)
    ver = a8.load_library().a8_version().decode()
    assert ver.endswith("src:" + bl.source_hash()), (ver, bl.source_hash())


def test_library_exports_every_declared_symbol(a8):
    lib = a8.load_library()
    raw = ctypes.CDLL(a8.LIB_PATH)
    for name in declared_functions():
        assert hasattr(raw, name), name
    assert lib.a8_version().decode().startswith("a8attn")
    assert "libamdhip64" in lib.a8_hip_runtime_path().decode()
    from audio8_turbo_engine_amd import _lib
    assert set(_lib.SIGNATURES) == set(declared_functions())


def _store_args(**kw):
    a = dict(qkv=16, s_qkv=1152, bias=None, cos=16, sin=16, s_cs=64, n_tab=8, pos=16, slot=16, R=1, qo=16,
             s_qo_r=896, s_qo_h=64, kc=16, vc=16, s_kb=1024, s_kh=512, s_ks=64, rows=1, S=8, nq=14, nkv=2, hd=64,
             ring=1 << 30, stream=None)
    a.update(kw)
    return list(a.values())


def test_store_rejects_before_launch(a8):
    lib = a8.load_library()
    assert lib.a8_bias_rope_store(*_store_args(hd=72)) == -3          # not a multiple of 16
    assert b"head_dim 72" in lib.a8_last_error()
    assert lib.a8_bias_rope_store(*_store_args(hd=512)) == -3
    assert lib.a8_bias_rope_store(*_store_args(ring=0)) == -1
    assert lib.a8_bias_rope_store(*_store_args(qkv=24)) == -2          # misaligned pointer
    assert lib.a8_bias_rope_store(*_store_args(s_qkv=1151)) == -2      # stride not a multiple of 8
    assert lib.a8_bias_rope_store(*_store_args(kc=None)) == -1         # (qo may be null: k / v only)
    assert lib.a8_bias_rope_store(*_store_args(R=0)) == 0              # nothing to do, nothing launched


def _decode_args(**kw):
    a = dict(q=16, s_qb=896, s_qh=64, kc=16, vc=16, s_kb=1024, s_kh=512, s_ks=64, rows=1, S=8, lens=16,
             rowmap=None, out=16, s_ob=896, s_oh=64, acc=16, ml=16, ws=4, counters=None, n_counters=0, b=1, nq=14,
             nkv=2, hd=64, nsplit=1, waves=4, scale=0.125, phases=3, stream=None)
    a.update(kw)
    return list(a.values())


def test_decode_rejects_before_launch(a8):
    lib = a8.load_library()
    assert lib.a8_decode_attn(*_decode_args(hd=96)) == -3               # 64 or 128
    assert lib.a8_decode_attn(*_decode_args(nq=34, nkv=2)) == -3        # group 17 > 16
    assert lib.a8_decode_attn(*_decode_args(nq=15)) == -1               # nq not a multiple of nkv
    assert lib.a8_decode_attn(*_decode_args(waves=3)) == -1
    assert lib.a8_decode_attn(*_decode_args(nsplit=0)) == -1
    assert lib.a8_decode_attn(*_decode_args(b=3, nsplit=2, ws=5)) == -4  # workspace: 6 row-splits needed
    assert lib.a8_decode_attn(*_decode_args(out=8)) == -2
    assert lib.a8_decode_attn(*_decode_args(b=0)) == 0
    # the in-kernel merge: one counter per (row, kv head), and the split kernel must run
    assert lib.a8_decode_attn(*_decode_args(b=3, nsplit=2, ws=6, counters=16, n_counters=5)) == -4
    assert b"counters" in lib.a8_last_error()
    assert lib.a8_decode_attn(*_decode_args(nsplit=2, ws=4, counters=16, n_counters=2, phases=2)) == -1


def test_fused_decode_refuses_other_head_dims(a8):
    """The fused store + decode kernels are head_dim 64 only: 128 is refused before any launch (callers make
    the two calls, as DecodeAttention.store_and_attend does)."""
    lib = a8.load_library()
    store = [16, 1152, None, 16, 16, 64, 8, 16, 16, None, 896, 64]
    dec = [16, 16, 1024, 512, 128, 1, 8, 16, None, 16, 896, 64, 16, 16, 4]
    st = lib.a8_store_decode_split(*store, *dec, None, 0, 1, 14, 2, 128, 1 << 30, 1, 4, 0.125, 3, None)
    assert st == -3 and b"head_dim 128" in lib.a8_last_error()


def _prefill_args(**kw):
    a = dict(q=16, s_qr=896, s_qh=64, R=4, kc=16, vc=16, s_kb=1024, s_kh=512, s_ks=64, rows=1, S=8, out=16,
             s_or=896, s_oh=64, bq0=16, bn=16, bslot=16, bpos0=16, nblk=1, bm=64, nq=14, group=7, hd=64,
             scale=0.125, stream=None)
    a.update(kw)
    return list(a.values())


def test_prefill_rejects_before_launch(a8):
    lib = a8.load_library()
    assert lib.a8_prefill_attn(*_prefill_args(bm=32)) == -3
    assert lib.a8_prefill_attn(*_prefill_args(hd=80)) == -3
    assert lib.a8_prefill_attn(*_prefill_args(group=5)) == -1
    assert lib.a8_prefill_attn(*_prefill_args(s_qr=900)) == -2
    assert lib.a8_prefill_attn(*_prefill_args(nblk=0)) == 0


def _prefill_qkv_args(**kw):
    a = dict(qkv=16, s_qkv=1152, bias=None, cos=16, sin=16, s_cs=64, n_tab=8, R=4, kc=16, vc=16, s_kb=1024,
             s_kh=512, s_ks=64, rows=1, S=8, out=16, s_or=896, s_oh=64, bq0=16, bn=16, bslot=16, bpos0=16,
             nblk=1, bm=64, nq=14, group=7, hd=64, scale=0.125, stream=None)
    a.update(kw)
    return list(a.values())


def test_prefill_qkv_rejects_before_launch(a8):
    """a8_prefill_attn_qkv refuses what a8_prefill_attn refuses, head_dim 128 (64 only), a missing table,
    misaligned, short or oversized tables before any launch."""
    lib = a8.load_library()
    f = lib.a8_prefill_attn_qkv
    assert f(*_prefill_qkv_args(bm=32)) == -3
    assert f(*_prefill_qkv_args(hd=128)) == -3 and b"head_dim 128" in lib.a8_last_error()
    assert f(*_prefill_qkv_args(group=5)) == -1
    assert f(*_prefill_qkv_args(cos=None)) == -1
    assert f(*_prefill_qkv_args(sin=24)) == -2
    assert f(*_prefill_qkv_args(s_cs=68)) == -2                 # not a multiple of 8
    assert f(*_prefill_qkv_args(s_cs=56)) == -1                 # rows shorter than head_dim
    assert f(*_prefill_qkv_args(n_tab=-1)) == -1
    assert f(*_prefill_qkv_args(n_tab=1 << 25)) == -3           # tables past 32-bit byte offsets
    assert f(*_prefill_qkv_args(nblk=0)) == 0


def _choose(lib, b, nkv=2, S=2048, req=1, nmax=16, cap=8192, n_cu=256):
    ns, nw = ctypes.c_int(), ctypes.c_int()
    assert lib.a8_decode_choose(b, nkv, S, req, nmax, cap, n_cu, ctypes.byref(ns), ctypes.byref(nw)) == 0
    return ns.value, nw.value


def test_decode_choose_contract(a8):
    lib = a8.load_library()
    for b in (1, 2, 4, 16, 64, 128, 192, 384, 1000):
        for S in (2, 10, 64, 385, 2048, 4096):
            for req in (1, 3, 16):
                for nmax in (1, 4, 16):
                    for cap in (b, 2 * b, 16 * b, 8192):
                        ns, nw = _choose(lib, b, S=S, req=req, nmax=nmax, cap=cap)
                        assert ns >= 1 and nw in (1, 2, 4, 8)
                        assert ns <= nmax and b * ns <= max(cap, b)
                        assert ns <= max(1, -(-S // 64))            # no more splits than 64-key tiles
                        if ns < req:                                 # only the caps may cut the request
                            assert ns in (nmax, cap // b, max(1, -(-S // 64)))
    # the peak-load config: one split (no combine launch), 4 waves per split
    assert _choose(lib, 192) == (1, 4)
    # a single row over a long cache is split to occupy the GPU
    ns, nw = _choose(lib, 1, S=2048)
    assert ns >= 4 and ns * nw * 2 <= 2 * 256 * 4
    # tiny caches: one wave, one split
    assert _choose(lib, 384, S=10, nmax=1) == (1, 1)
    with pytest.raises(ctypes.ArgumentError):
        lib.a8_decode_choose(1, 2, 8, 1, 1, 8, 256, None, "x")
    assert lib.a8_decode_choose(0, 2, 8, 1, 1, 8, 256, ctypes.byref(ctypes.c_int()), ctypes.byref(ctypes.c_int())) == -1


def _stream_args(**kw):
    a = dict(q=16, s_qb=896, s_qh=64, kc=16, vc=16, s_kb=1024, s_kh=512, s_ks=64, rows=1, S=8, lens=16,
             rowmap=None, out=16, s_ob=896, s_oh=64, acc=16, ml=16, ws=4, b=1, nq=14, nkv=2, hd=64,
             waves=4, tpw=2, grid=4, scale=0.125, phases=3, stream=None)
    a.update(kw)
    return list(a.values())


def test_decode_stream_rejects_before_launch(a8):
    lib = a8.load_library()
    f = lib.a8_decode_attn_stream
    assert f(*_stream_args(hd=32)) == -3
    assert f(*_stream_args(nq=34)) == -3
    assert f(*_stream_args(waves=5)) == -1
    assert f(*_stream_args(waves=8)) == -3                          # LDS: 1, 2 or 4 waves
    assert f(*_stream_args(tpw=0)) == -1
    assert f(*_stream_args(grid=0)) == -1
    # 3 rows over a 2048-key cache in 512-key chunks need 3 * 4 row-splits of workspace
    assert f(*_stream_args(b=3, S=2048, ws=11)) == -4
    assert f(*_stream_args(b=3, S=2048, ws=12, ml=None)) == -4
    assert f(*_stream_args(q=8)) == -2
    assert f(*_stream_args(b=0)) == 0


def _choose_stream(lib, b, nkv=2, S=2048, cap=8192, n_cu=256):
    nw, tpw, grid = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    assert lib.a8_decode_choose_stream(b, nkv, S, cap, n_cu, ctypes.byref(nw), ctypes.byref(tpw),
                                       ctypes.byref(grid)) == 0
    return nw.value, tpw.value, grid.value


def test_decode_choose_stream_contract(a8):
    lib = a8.load_library()
    for b in (1, 2, 16, 64, 192, 384, 2000):
        for S in (1, 10, 64, 385, 2048, 4096):
            for cap in (b, 4 * b, 16 * b, 8192):
                nw, tpw, grid = _choose_stream(lib, b, S=S, cap=cap)
                assert nw in (1, 2, 4, 8) and tpw >= 1 and grid >= 1
                ch = nw * tpw * 64
                P = -(-S // ch)
                assert P == 1 or b * P <= cap or tpw >= 64     # fits the workspace
                assert grid <= b * 2 * P                          # no idle workgroups
    # the peak-load config: whole-unit chunks, two per workgroup of 4 waves on 192 workgroups
    assert _choose_stream(lib, 192) == (4, 8, 192)
    # tiny caches: one wave, one tile, four units per workgroup
    assert _choose_stream(lib, 384, S=10, cap=384) == (1, 1, 192)
    # a single long row is cut into chunks to occupy the GPU
    nw, tpw, grid = _choose_stream(lib, 1, S=2048)
    assert -(-2048 // (nw * tpw * 64)) >= 8 and grid >= 8


def _flat_args(**kw):
    a = dict(q=16, s_qb=896, s_qh=64, kc=16, vc=16, s_kb=1024, s_kh=512, s_ks=64, rows=4, S=8, lens=16, rowmap=None,
             out=16, s_ob=896, s_oh=64, acc=16, ml=16, ws=64, cnt=16, ncnt=8, b=4, nq=14, nkv=2, hd=64, grid=4,
             scale=0.125, stream=None)
    a.update(kw)
    return list(a.values())


def _store_flat_args(**kw):
    a = dict(qkv=16, s_qkv=1152, bias=None, cos=16, sin=16, s_cs=64, n_tab=8, pos=16, slot=16, qo=None, s_qo_r=0,
             s_qo_h=0, kc=16, vc=16, s_kb=1024, s_kh=512, s_ks=64, rows=4, S=8, lens=16, rowmap=None, out=16,
             s_ob=896, s_oh=64, acc=16, ml=16, ws=64, cnt=16, ncnt=8, b=4, nq=14, nkv=2, hd=64, ring=1 << 30, grid=4,
             scale=0.125, stream=None)
    a.update(kw)
    return list(a.values())


def test_decode_flat_rejects_before_launch(a8):
    """Every call here fails its argument checks (or has no rows), so nothing is launched."""
    lib = a8.load_library()
    f = lib.a8_decode_attn_flat
    assert f(*_flat_args(hd=32)) == -3
    assert f(*_flat_args(nq=34)) == -3                               # GQA group 17
    assert f(*_flat_args(b=2049, ncnt=8192)) == -3                   # rows per call (metadata in LDS)
    assert b"2049 rows" in lib.a8_last_error()
    assert f(*_flat_args(grid=0)) == -1
    assert f(*_flat_args(cnt=None)) == -1
    assert f(*_flat_args(grid=17, ws=67)) == -4                      # 2 slots per wave: 136 > 67 * 2
    assert f(*_flat_args(ncnt=7)) == -4                              # b * nkv counters
    assert f(*_flat_args(q=8)) == -2
    assert f(*_flat_args(s_oh=60)) == -2
    assert f(*_flat_args(s_ks=128)) == -3
    assert f(*_flat_args(b=0)) == 0
    g = lib.a8_store_decode_flat
    assert g(*_store_flat_args(ring=0)) == -1
    assert g(*_store_flat_args(pos=None)) == -1
    assert g(*_store_flat_args(qkv=24)) == -2
    assert g(*_store_flat_args(nq=30)) == -3                         # group 15: lanes 14 / 15 hold k / v
    assert g(*_store_flat_args(ncnt=7)) == -4
    assert g(*_store_flat_args(b=0)) == 0


def _choose_flat(lib, b, nkv=2, S=2048, cap=8192, n_cu=256):
    grid = ctypes.c_int()
    st = lib.a8_decode_choose_flat(b, nkv, S, cap, n_cu, ctypes.byref(grid))
    return st, grid.value


def test_decode_choose_flat_contract(a8):
    lib = a8.load_library()
    for b in (1, 2, 16, 64, 192, 384, 2000):
        for S in (1, 10, 64, 385, 2048, 4096):
            for cap in (b, 4 * b, 16 * b, 8192):
                st, grid = _choose_flat(lib, b, S=S, cap=cap)
                if cap * 2 < 8:                                      # not even one workgroup's slots
                    assert st == -4
                    continue
                assert st == 0 and 1 <= grid <= 256
                assert 2 * grid * 4 <= cap * 2                       # two partial slots per wave fit
                assert grid * 4 <= max(4, b * 2 * -(-S // 64) + 3)   # no more waves than tiles (rounded up)
    assert _choose_flat(lib, 1, S=512) == (0, 4)                     # C1: 16 tiles, one per wave
    assert _choose_flat(lib, 64, S=4096) == (0, 256)                 # C2: the whole GPU
    assert _choose_flat(lib, 384, S=10, cap=384) == (0, 96)          # C5 (fast stack workspace)



def _prefix_args(**kw):
    a = dict(k=16, v=16, s_l=2 * 300 * 64, s_h=300 * 64, s_p=64, kc=16, vc=16, d_l=70 * 2 * 704 * 64,
             d_r=2 * 704 * 64, d_h=704 * 64, d_p=64, slots=16, n=4, layers=24, nkv=2, Lp=300, hd=64, rows=70, S=704,
             stream=None)
    a.update(kw)
    return list(a.values())


def test_prefix_copy_rejects_before_launch(a8):
    lib = a8.load_library()
    assert lib.a8_prefix_copy(*_prefix_args(hd=128)) == -3
    assert lib.a8_prefix_copy(*_prefix_args(Lp=705)) == -1          # the prefix does not fit the cache
    assert b"705" in lib.a8_last_error()
    assert lib.a8_prefix_copy(*_prefix_args(s_p=128)) == -3         # positions must be contiguous rows
    assert lib.a8_prefix_copy(*_prefix_args(k=24)) == -2            # misaligned
    assert lib.a8_prefix_copy(*_prefix_args(d_r=100)) == -2         # stride not a multiple of 8
    assert lib.a8_prefix_copy(*_prefix_args(slots=None)) == -1
    assert lib.a8_prefix_copy(*_prefix_args(n=-1)) == -1
    for zero in (dict(n=0), dict(layers=0), dict(Lp=0)):
        assert lib.a8_prefix_copy(*_prefix_args(**zero)) == 0     # nothing to do, nothing launched


def test_layer_ops_reject_before_launch(a8):
    lib = a8.load_library()
    args = dict(x=16, sx=896, r=None, sr=0, w=16, y=16, sy=896, ro=None, sro=0, rows=4, N=896, eps=1e-6, stream=None)
    assert lib.a8_rmsnorm(*{**args, "N": 900}.values()) == -3               # not a multiple of 8
    assert lib.a8_rmsnorm(*{**args, "N": 4096}.values()) == -3              # wider than 2048
    assert lib.a8_rmsnorm(*{**args, "r": 16}.values()) == -1                # a residual needs res_out
    assert lib.a8_rmsnorm(*{**args, "x": 24}.values()) == -2
    assert lib.a8_rmsnorm(*{**args, "rows": 0}.values()) == 0
    assert lib.a8_silu_mul(16, 2048, 16, 1024, 4, 1020, None) == -3
    assert lib.a8_silu_mul(16, 2047, 16, 1024, 4, 1024, None) == -2
    assert lib.a8_silu_mul(None, 2048, 16, 1024, 4, 1024, None) == -1
    assert lib.a8_silu_mul(16, 2048, 16, 1024, 0, 1024, None) == 0


def test_conv_ops_reject_before_launch(a8):
    lib = a8.load_library()
    conv = dict(x=16, s_xb=10 * 64, s_xt=64, w=16, s_wp=7 * 64 * 64, s_wt=64 * 64, s_wc=64, cout_w=64, bias=None,
                res=None, s_rb=0, s_rt=0, y=16, s_yb=4 * 64, s_yt=64, sa=None, sib=None, B=2, Tin=10, TR=4, Cin=64,
                Cout=64, taps=7, dil=1, ph=1, ws=None, nws=0, stream=None)
    assert lib.a8_conv_cl(*{**conv, "Tin": 9}.values()) == -1           # 4 + 6 context rows needed
    assert b"input rows" in lib.a8_last_error()
    assert lib.a8_conv_cl(*{**conv, "Cin": 60}.values()) == -3          # channels in 16-byte chunks
    assert lib.a8_conv_cl(*{**conv, "cout_w": 32}.values()) == -1       # the weights hold fewer columns
    assert lib.a8_conv_cl(*{**conv, "sa": 16}.values()) == -1           # snake needs both vectors
    assert lib.a8_conv_cl(*{**conv, "sa": 16, "sib": 16, "Cin": 1032, "s_xt": 1032, "s_wt": 1032 * 64,
                            "s_xb": 10 * 1032}.values()) == -3               # snake on the load: Cin <= 1024
    assert b"snake" in lib.a8_last_error()
    assert lib.a8_conv_cl(*{**conv, "x": 24}.values()) == -2
    assert lib.a8_conv_cl(*{**conv, "TR": 0, "Tin": 6}.values()) == 0
    # split-K workspace: short inputs with long K get one, long inputs none
    assert lib.a8_conv_cl_ws_bytes(192, 4, 1024, 1536, 7, 1) > 0
    assert lib.a8_conv_cl_ws_bytes(192, 1024, 192, 192, 7, 1) == 0
    assert lib.a8_conv_cl_ws_bytes(0, 4, 1024, 1536, 7, 1) == 0
    snake = dict(x=16, s_xb=5 * 64, s_xt=64, st=16, s_sb=3 * 64, s_st=64, a=None, ib=None, y=16, s_yb=8 * 64, s_yt=64,
                 B=2, T=5, CTX=3, C=64, stream=None)
    assert lib.a8_snake_cat(*{**snake, "C": 60}.values()) == -3
    assert lib.a8_snake_cat(*{**snake, "st": None}.values()) == -1
    assert lib.a8_snake_cat(*{**snake, "s_yt": 60}.values()) == -2
    assert lib.a8_snake_cat(*{**snake, "B": 0}.values()) == 0
