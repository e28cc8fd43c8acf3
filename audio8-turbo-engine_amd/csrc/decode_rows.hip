// Whole-row decode: the launch a8_decode_attn_stream / a8_store_decode_stream make when one chunk holds a
// whole row at 4 waves and one tile per step (the peak-load shape, 192 rows x 2048 keys). Same work per
// wave as k_decode_stream with one chunk per unit -- wave w of the workgroup consumes tiles w, w + 4, ...
// of the unit (row, kv head) with decode_tile.h's step, and the last wave to finish merges the four
// partials with the same arithmetic -- so the results are the same bits. Semantics are those of
// serve/fast_kernels.py:193-290 (and, fused, bias_rope_store of 139-187 first).
//
// What differs is the timeline around each unit (measured with per-wave clock stamps on MI355X: a unit
// transition cost every wave ~1.3 us, the last unit's merge ~1.4 us, and the first q was ready ~2.9 us
// after the first tile request, its RoPE-table loads queued behind every wave's first tiles):
//   * Workgroup g takes units g, g + G, ...; a unit's SPW steps are unrolled, so every load, store and
//     wait sits at a fixed point and the compiler's wait counts are exact (no branch joins paths with
//     different numbers of memory operations in flight). Stores that only some lanes or waves make are
//     buffer stores whose range check drops the others' (no branch around them either).
//   * The inputs of unit i + 1 (q, or its qkv / bias / RoPE-table rows) are requested at unit i's first
//     step and, fused, rotated at its fourth, when they have long arrived; the k / v / q store of unit
//     i + 1 goes out then too. The metadata of unit i + 2 follows at unit i's first step. At the
//     transition no wave waits for anything but its next tile.
//   * The first unit's metadata and qkv / bias rows go out before any tile, its table rows as soon as the
//     position returns and before the tiles, so q is ready about when the first tiles land.
//   * The merge reads every parked partial it needs with one batch of LDS reads.
//   * Nothing is requested past the last tile (the pipeline's last two steps issue no load).
// Measured at 192 rows x 2048 keys, 24 layers in a graph: 36.2-36.9 us per layer unfused and 37.5-38.1
// fused (store included), against 37.2-37.8 and 39.3-39.7 for k_decode_stream on the same boxes. Tried and
// slower: four tiles in flight per wave (+1 us), the first tiles requested before the position (+0.9 to
// +2.3 us: the table rows then return behind them, also when read through the scalar cache), the unit
// park deferred behind the next unit's first request (+0.3 us); the order of the tiles within a unit and
// of the units over the workgroups changed nothing beyond box-to-box noise.
#include "fused_qkv.h"

namespace a8 {

namespace {

constexpr int kRowsNW = 4;
constexpr uint32_t kOOR = 0xFFFFFF00u;  // buffer offset past any range: the access is dropped

__device__ __forceinline__ void bst16(rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, 0);
}
__device__ __forceinline__ void bst8(rsrc_t r, uint32_t off, u32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, (int)off, 0, 0);
}

// Per-unit metadata, requested ahead (vector loads: they complete in order with the tile loads).
struct RowMeta {
  int craw, lraw, praw, sraw;  // row map entry, length, position, slot
};

struct RowUnit {
  int row, kh, hi;  // keys [0, hi) of cache row crow are attended
  int crow;
  rsrc_t kr, vr;
};

}  // namespace

template <bool FUSED, int SPW>
__global__ __launch_bounds__(64 * kRowsNW, 1) void k_decode_rows(
    const uint16_t *__restrict__ q, int64_t s_qb, int64_t s_qh,
    uint16_t *kc, uint16_t *vc, int64_t s_kb, int64_t s_kh,
    int cache_rows, int cache_len, const int32_t *__restrict__ lens, const int32_t *__restrict__ rowmap,
    uint16_t *__restrict__ out, int64_t s_ob, int64_t s_oh, int b, int nq, int nkv, int group,
    float sl2, StoreIn si) {
  constexpr int NW = kRowsNW;
  // tiles in flight per wave: two (measured on MI355X at the peak load: four in flight per wave ran ~1 us per
  // layer slower, the deeper queues costing more than they hide)
  constexpr int D = 2;
  warm_kernargs<232>();  // the explicit arguments above span 0x00-0xe7
  static_assert(SPW % D == 0 && SPW >= 4, "steps per unit");
  // V tiles of the two pipeline buffers: separate arrays, so the compiler tells their DMA completions apart and
  // waits only for the buffer it reads
  __shared__ __attribute__((aligned(16))) uint16_t vb0[NW * kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t vb1[NW * kVTile];
  // per-wave m, l, O of a finished unit, two areas (a unit's merge may still read one while the next parks)
  constexpr int MB = 2;
  __shared__ __attribute__((aligned(16))) float mrg[MB][NW * (32 + 16 * kOb)];
  __shared__ int marr[MB], mseq[MB];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x;
  const int U = b * nkv;
  const int nmine = ((int)blockIdx.x < U) ? (U - 1 - (int)blockIdx.x) / G + 1 : 0;
  if (nmine == 0) return;
  if (tid < MB) {
    marr[tid] = 0;
    mseq[tid] = tid - MB;
  }
  lds_barrier();

  TileLane tl;
  tl.init(lane);
  uint16_t *const vbw[2] = {vb0 + w * kVTile, vb1 + w * kVTile};

  // ---- metadata, inputs and the tile sources of unit i (i >= nmine: empty ranges, nothing is read) ----
  const rsrc_t lens_r = make_rsrc(lens, (uint32_t)b * 4u);
  const rsrc_t map_r = make_rsrc(rowmap, rowmap ? (uint32_t)b * 4u : 0u);
  const rsrc_t pos_r = make_rsrc(si.pos, FUSED ? (uint32_t)b * 4u : 0u);
  const rsrc_t slot_r = make_rsrc(si.slot, FUSED ? (uint32_t)b * 4u : 0u);
  auto unit_of = [&](int i) { return (int)blockIdx.x + i * G; };
  auto tile_of = [&](int j) { return w + NW * j; };  // wave w: tiles w, w + NW, ... of the unit
  auto row_of = [&](int i) { return unit_of(i) / nkv; };
  auto meta_load = [&](int i) {
    const bool live = i < nmine;
    const uint32_t o = (uint32_t)(live ? row_of(i) : 0) * 4u;
    const uint32_t dead = live ? 0u : kOOR;  // past the range: reads 0 without memory traffic
    RowMeta m;
    m.craw = bld4(map_r, o + dead);  // without a row map an empty range (no branch around the load)
    m.lraw = bld4(lens_r, o + dead);
    m.praw = FUSED ? bld4(pos_r, o + dead) : 0;
    m.sraw = FUSED ? bld4(slot_r, o + dead) : 0;
    return m;
  };
  // exact = false: the range is the whole cache row (the length is not waited for; hi is set later)
  auto resolve = [&](int i, const RowMeta &m, RowUnit &un, bool exact) {
    const int u = unit_of(i);
    un.row = u / nkv;
    un.kh = u - un.row * nkv;
    int crow = un.row;
    if (rowmap) crow = __builtin_amdgcn_readfirstlane(m.craw);  // waits for the row map only when there is one
    const bool ok = i < nmine && crow >= 0 && crow < cache_rows;
    un.crow = ok ? crow : -1;
    un.hi = (ok && exact) ? min(max(__builtin_amdgcn_readfirstlane(m.lraw), 0), cache_len) : 0;
    const int64_t cb = (int64_t)(ok ? crow : 0) * s_kb + (int64_t)un.kh * s_kh;
    const uint32_t bound = ok ? (uint32_t)(exact ? un.hi : cache_len) * kRow : 0u;
    un.kr = make_rsrc_wave(kc + cb, bound);
    un.vr = make_rsrc_wave(vc + cb, bound);
  };
  // unfused: the unit's q rows (lanes r16 < group: q head kh * group + r16)
  auto load_q = [&](const RowUnit &un, bool live, u32x4 &q0, u32x4 &q1) {
    const rsrc_t qr = make_rsrc(q + (int64_t)(live ? un.row : 0) * s_qb + (int64_t)un.kh * group * s_qh,
                                live ? (uint32_t)(group * s_qh * 2) : 0u);
    const uint32_t qo = (uint32_t)(tl.r16 * s_qh * 2) + 16u * tl.g;
    q0 = bld16(qr, qo);
    q1 = bld16(qr, qo + 64u);
  };

  // fused: qkv / bias chunks (lane head: fused_lane_head) and the position's table chunks
  auto load_xb = [&](const RowUnit &un, bool live, QkvRaw &r) {
    const int H = nq + 2 * nkv;
    const rsrc_t xr = make_rsrc_wave(si.qkv + (int64_t)(live ? un.row : 0) * si.s_qkv, live ? (uint32_t)H * 128u : 0u);
    const rsrc_t br = make_rsrc(si.bias, (si.bias && live) ? (uint32_t)H * 128u : 0u);
    const uint32_t ho = (uint32_t)fused_lane_head(tl.r16, un.kh, group, nq, nkv) * 128u + 16u * tl.g;
    r.w[0] = bld16(xr, ho);
    r.w[1] = bld16(xr, ho + 64u);
    r.bb[0] = bld16(br, ho);
    r.bb[1] = bld16(br, ho + 64u);
  };
  auto load_tab = [&](bool live, int p, QkvRaw &r) {
    const bool pv = live && p >= 0 && p < si.n_tab;
    const rsrc_t cr = make_rsrc_wave(si.cos_tab + (int64_t)(pv ? p : 0) * si.s_cs, pv ? 128u : 0u);
    const rsrc_t sr = make_rsrc_wave(si.sin_tab + (int64_t)(pv ? p : 0) * si.s_cs, pv ? 128u : 0u);
    const uint32_t og = 16u * tl.g;
    r.cs[0] = bld16(cr, og);
    r.cs[1] = bld16(cr, og + 64u);
    r.sn[0] = bld16(sr, og);
    r.sn[1] = bld16(sr, og + 64u);
  };
  // fused: one RoPE pass per lane (rope.h arithmetic) -> the unit's Q^T operands and its patch column (the new
  // key, when the row attends the cache row it stores into); the k / v / q rows bias_rope_store writes are
  // pt.lo / pt.hi of the lanes kLaneK / kLaneV / r16 < group (rope_store).
  struct StoreDst {
    rsrc_t kr, vr, qr;
    uint32_t ko, vo, qo;
  };
  auto rope_unit = [&](const RowUnit &un, bool live, int p, int srow, const QkvRaw &r, u32x4 &q0, u32x4 &q1,
                       KVPatch &pt, StoreDst &sd) {
    const bool pv = live && p >= 0 && p < si.n_tab;
    const int sidx = pv ? p % si.ring : 0;
    const bool store_ok = pv && srow >= 0 && srow < cache_rows && sidx < cache_len;
    float xl[8], xh[8], ol[8], oh[8];
    rope_x(r.w[0], r.w[1], r.bb[0], r.bb[1], si.bias != nullptr, xl, xh);
    rope_rotate_f(xl, xh, r.cs[0], r.cs[1], r.sn[0], r.sn[1], ol, oh);
    const bool vlane = tl.r16 == kLaneV, klane = tl.r16 == kLaneK;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ol[j] = vlane ? xl[j] : ol[j];
      oh[j] = vlane ? xh[j] : oh[j];
    }
    rope_narrow(ol, oh, pt.lo, pt.hi);
    const bool qlive = pv && tl.r16 < group;
    const u32x4 z{0u, 0u, 0u, 0u};
    q0 = qlive ? pt.lo : z;
    q1 = qlive ? pt.hi : z;
    pt.col = (store_ok && srow == un.crow) ? sidx : -1;
    // stores from wave 0 only; every lane of every wave issues them and the range check drops the others'
    const bool w0 = w == 0;
    const int64_t kvo = (int64_t)(store_ok ? srow : 0) * s_kb + (int64_t)un.kh * s_kh + (int64_t)sidx * 64;
    sd.kr = make_rsrc_wave(kc + kvo, store_ok ? 128u : 0u);
    sd.vr = make_rsrc_wave(vc + kvo, store_ok ? 128u : 0u);
    const bool qw = si.qo != nullptr && pv;
    sd.qr = make_rsrc_wave(si.qo + (int64_t)(qw ? un.row : 0) * si.s_qo_r + (int64_t)un.kh * group * si.s_qo_h,
                           qw ? (uint32_t)((group - 1) * si.s_qo_h * 2 + 128) : 0u);
    const uint32_t og = 16u * tl.g;
    sd.ko = (w0 && klane) ? og : kOOR;
    sd.vo = (w0 && vlane) ? og : kOOR;
    sd.qo = (w0 && tl.r16 < group) ? (uint32_t)(tl.r16 * si.s_qo_h * 2) + og : kOOR;
  };
  auto rope_store = [&](const KVPatch &pt, const StoreDst &sd) {
    bst16(sd.kr, sd.ko, pt.lo);
    bst16(sd.kr, sd.ko + 64u, pt.hi);
    bst16(sd.vr, sd.vo, pt.lo);
    bst16(sd.vr, sd.vo + 64u, pt.hi);
    bst16(sd.qr, sd.qo, pt.lo);
    bst16(sd.qr, sd.qo + 64u, pt.hi);
  };

  SoftmaxState S;
  S.reset();
  KTile T0[1], T1[1];
  RowUnit cur, nxt;
  u32x4 qc0, qc1, qn0, qn1;
  KVPatch ptc, ptn;
  ptc.col = -1;
  ptn.col = -1;
  QkvRaw rn;      // fused: raw chunks of the next unit, between its request and its rotation
  StoreDst sdn;   // fused: where unit 0's / the next unit's k / v / q go
  int mcur_p = 0, mcur_s = 0;  // fused: position / slot of unit i + 1 while it is prepared

  // ---- unit finish: park, count in; the last of the NW waves merges and writes out ----
  int nfin = 0;
  auto finish = [&](const RowUnit &un) {
    const int n = nfin++;
    const int bsel = MB > 1 ? (n & 1) : 0;
    float *mb = mrg[bsel], *lb = mb + NW * 16, *ob = mb + NW * 32;
    const float lsum = sum_over_groups(S.lsum);
    // the merge of unit n - MB out of this area is complete (it waits for nothing, so this ends; bounded all
    // the same)
    for (int spin = 0; spin < (1 << 22) && lds_read_word(&mseq[bsel]) < n - MB; ++spin) __builtin_amdgcn_s_sleep(1);
    if (tl.g == 0) {
      mb[w * 16 + tl.r16] = S.m;
      lb[w * 16 + tl.r16] = lsum;
    }
    lds_store_4x16(ob + (w * 16 + tl.r16) * kOb + 4 * tl.g, S.o[0], S.o[1], S.o[2], S.o[3]);
    S.reset();
    const bool last = lds_add_word(&marr[bsel], 1) == NW - 1;
    // the output row of the unit: lanes (head, 4 dims), item t = lane and lane + 64 (t < group * 16)
    const rsrc_t orr = make_rsrc_wave(out + (int64_t)un.row * s_ob + (int64_t)un.kh * group * s_oh,
                                      (uint32_t)(((group - 1) * s_oh + 64) * 2));
    u32x2 res[2];
    uint32_t ooff[2];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      res[it] = u32x2{0u, 0u};
      ooff[it] = kOOR;
    }
    if (last) {
      lds_write_word(&marr[bsel], 0);  // the buffer's next arrivals come after mseq says n is merged
      float mv[2][NW], lv[2][NW];
      f32x4 ov[2][NW];
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int t = min(lane + 64 * it, group * 16 - 1);
        const int head = t >> 4, d4 = (t & 15) * 4;
#pragma unroll
        for (int v = 0; v < NW; ++v) {
          mv[it][v] = mb[v * 16 + head];
          lv[it][v] = lb[v * 16 + head];
          ov[it][v] = *reinterpret_cast<const f32x4 *>(ob + (v * 16 + head) * kOb + d4);
        }
      }
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int t = lane + 64 * it;
        const int head = t >> 4, d4 = (t & 15) * 4;
        float M = kNegInf;
#pragma unroll
        for (int v = 0; v < NW; ++v) M = fmaxf(M, mv[it][v]);
        f32x4 num = {0.f, 0.f, 0.f, 0.f};
        float den = 0.f;
#pragma unroll
        for (int v = 0; v < NW; ++v) {
          const float wt = (mv[it][v] == kNegInf) ? 0.f : fast_exp2((mv[it][v] - M) * sl2);
          num += wt * ov[it][v];
          den += wt * lv[it][v];
        }
        res[it][0] = pack_bf16x2(num[0] / den, num[1] / den);
        res[it][1] = pack_bf16x2(num[2] / den, num[3] / den);
        if (t < group * 16) ooff[it] = (uint32_t)(head * s_oh * 2 + d4 * 2);
      }
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) bst8(orr, ooff[it], res[it]);
    if (last) lds_write_word(&mseq[bsel], n);  // after the reads above: the buffer may be reused
  };

  // ---- steps: compute tile j of the current unit from buffer j % D, then request into it tile j + D of the
  // unit, or tile j + D - SPW of the next (one load sequence, sources selected) ----
  auto step = [&](KTile(&X)[1], uint16_t *xv, int j, bool reload) __attribute__((always_inline)) {
    const int t0 = 64 * tile_of(j);
    if (t0 < cur.hi) compute_step<1, FUSED>(X, xv, t0, cur.hi, qc0, qc1, sl2, S, tl, lane, &ptc);
    if (reload) {
      const bool in_cur = j + D < SPW;
      const rsrc_t kr = in_cur ? cur.kr : nxt.kr, vr = in_cur ? cur.vr : nxt.vr;
      const int jj = in_cur ? j + D : j + D - SPW;
      load_step<1>(X, xv, kr, vr, (uint32_t)(64 * tile_of(jj)), tl);
    }
  };
  auto step_k = [&](int j, bool reload) __attribute__((always_inline)) {
    if (j & 1)
      step(T1, vbw[1], j, reload);
    else
      step(T0, vbw[0], j, reload);
  };
  auto first_load = [&](int j) __attribute__((always_inline)) {
    const uint32_t t0 = (uint32_t)(64 * tile_of(j));
    if (j & 1)
      load_step<1>(T1, vbw[1], cur.kr, cur.vr, t0, tl);
    else
      load_step<1>(T0, vbw[0], cur.kr, cur.vr, t0, tl);
  };
  constexpr int kRopeStep = D < SPW - 1 ? D : SPW - 1;  // the next unit's inputs have arrived by then

  // ---- prologue: unit 0's metadata and q inputs go out before its first tile; unit 1's metadata with them ----
  RowMeta m0 = meta_load(0);
  RowMeta mn = meta_load(1);
  {
    RowUnit u0;
    u0.row = row_of(0);
    u0.kh = unit_of(0) - u0.row * nkv;
    QkvRaw r0;
    if (FUSED) {
      // the table rows go out as soon as the position is in, ahead of every tile (their data would return
      // behind the tiles' otherwise: measured slower with the first tile, or all, requested before the
      // position); the range is exact
      load_xb(u0, true, r0);
      load_tab(true, __builtin_amdgcn_readfirstlane(m0.praw), r0);
      resolve(0, m0, cur, true);
      first_load(0);
      // unit 0's rotation, once its table rows are in; its stores follow the first step
      rope_unit(cur, true, __builtin_amdgcn_readfirstlane(m0.praw), __builtin_amdgcn_readfirstlane(m0.sraw), r0, qc0,
                qc1, ptc, sdn);
#pragma unroll
      for (int j = 1; j < D; ++j) first_load(j);
    } else {
      // unfused: the first tiles go out over the whole cache row before the length returns; the range is
      // narrowed after them
      load_q(u0, true, qc0, qc1);
      resolve(0, m0, cur, false);
#pragma unroll
      for (int j = 0; j < D; ++j) first_load(j);
      resolve(0, m0, cur, true);
    }
  }

  // ---- units 0 .. nmine - 2: every step requests D tiles ahead, across into the next unit ----
  for (int i = 0; i < nmine - 1; ++i) {
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      if (j == 0) {
        // unit i + 1: its tile sources and inputs; unit i + 2's metadata
        resolve(i + 1, mn, nxt, true);
        if (FUSED) {
          mcur_p = __builtin_amdgcn_readfirstlane(mn.praw);
          mcur_s = __builtin_amdgcn_readfirstlane(mn.sraw);
          load_xb(nxt, true, rn);
          load_tab(true, mcur_p, rn);
        } else {
          load_q(nxt, true, qn0, qn1);
        }
        mn = meta_load(i + 2);
      }
      step_k(j, true);
      if (FUSED && j == 0 && i == 0) rope_store(ptc, sdn);  // unit 0's k / v / q
      if (FUSED && j == kRopeStep) {
        rope_unit(nxt, true, mcur_p, mcur_s, rn, qn0, qn1, ptn, sdn);
        rope_store(ptn, sdn);
      }
    }
    finish(cur);
    cur = nxt;
    qc0 = qn0;
    qc1 = qn1;
    if (FUSED) ptc = ptn;
  }
  // ---- the last unit: no request past its last tile ----
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    step_k(j, j + D < SPW);
    if (FUSED && j == 0 && nmine == 1) rope_store(ptc, sdn);
  }
  finish(cur);
}

template <bool FUSED, int SPW>
static void launch_rows(int grid, hipStream_t st, const uint16_t *q, int64_t s_qb, int64_t s_qh, uint16_t *kc,
                        uint16_t *vc, int64_t s_kb, int64_t s_kh, int cache_rows, int cache_len, const int32_t *lens,
                        const int32_t *rowmap, uint16_t *out, int64_t s_ob, int64_t s_oh, int b, int nq, int nkv,
                        int group, float sl2, const StoreIn &si) {
  hipLaunchKernelGGL((k_decode_rows<FUSED, SPW>), dim3(grid), dim3(64 * kRowsNW), 0, st, q, s_qb, s_qh, kc, vc, s_kb,
                     s_kh, cache_rows, cache_len, lens, rowmap, out, s_ob, s_oh, b, nq, nkv, group, sl2, si);
}

// Launches k_decode_rows when it serves the shape (whole rows per chunk at 4 waves x 1 tile per step, at
// most 16 steps per unit); returns false otherwise. Arguments are checked by the caller.
bool rows_launch(int grid, hipStream_t st, const uint16_t *q, int64_t s_qb, int64_t s_qh, uint16_t *kc, uint16_t *vc,
                 int64_t s_kb, int64_t s_kh, int cache_rows, int cache_len, const int32_t *lens, const int32_t *rowmap,
                 uint16_t *out, int64_t s_ob, int64_t s_oh, int b, int nq, int nkv, int group, float sl2,
                 const StoreIn &si) {
  const bool fused = si.qkv != nullptr;
  const int spw = (cache_len + 64 * kRowsNW - 1) / (64 * kRowsNW);
  const int SPW = spw <= 4 ? 4 : spw <= 8 ? 8 : spw <= 16 ? 16 : 0;
  if (SPW == 0 || spw < 2) return false;
#define A8_ROWS_ARGS grid, st, q, s_qb, s_qh, kc, vc, s_kb, s_kh, cache_rows, cache_len, lens, rowmap, out, s_ob, s_oh, \
                     b, nq, nkv, group, sl2, si
  switch (SPW * 2 + (fused ? 1 : 0)) {
    case 8: launch_rows<false, 4>(A8_ROWS_ARGS); break;
    case 9: launch_rows<true, 4>(A8_ROWS_ARGS); break;
    case 16: launch_rows<false, 8>(A8_ROWS_ARGS); break;
    case 17: launch_rows<true, 8>(A8_ROWS_ARGS); break;
    case 32: launch_rows<false, 16>(A8_ROWS_ARGS); break;
    default: launch_rows<true, 16>(A8_ROWS_ARGS); break;
  }
#undef A8_ROWS_ARGS
  return true;
}

}  // namespace a8
