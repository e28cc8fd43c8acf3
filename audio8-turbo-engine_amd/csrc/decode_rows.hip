// Whole-row decode: the launch a8_decode_attn_stream / a8_store_decode_stream make when one chunk holds a
// whole row at 4 waves and one tile per step (the peak-load shape, 192 rows x 2048 keys). Wave w of the
// workgroup consumes tiles w, w + 4, ... of the unit (row, kv head) with decode_tile.h's step; the four
// partials are merged with k_decode_combine's arithmetic. Semantics are those of serve/fast_kernels.py:193-290
// (and, fused, bias_rope_store of 139-187 first).
//
// The timeline around each unit (measured with per-wave clock stamps and with copies that skip parts of the
// work, on MI355X at 192 rows x 2048 keys):
//   * Workgroup g takes units g, g + G, ...; a unit's SPW steps are unrolled, so every load, store and
//     wait sits at a fixed point and the compiler's wait counts are exact (no branch joins paths with
//     different numbers of memory operations in flight). Stores that only some lanes or waves make are
//     buffer stores whose range check drops the others' (no branch around them either).
//   * Unit u starts at step u % SPW (its waves take their tiles in the same rotated order). Units whose
//     streams all start at the same offset and advance in step meet the same memory channels at the same
//     time: a plain read of the peak-load bytes in this kernel's pattern took 35.2 us with every unit starting
//     at key 0 and 33.6-33.8 us with the rotation; the decode itself gained 0.2-0.4 us.
//   * The inputs of unit i + 1 (q, or its qkv / bias / RoPE-table rows) are requested at unit i's first
//     step and, fused, rotated at its third, when they have long arrived. The metadata of unit i + 2
//     follows at unit i's first step. At the transition no wave waits for anything but its next tile.
//   * The first unit's metadata and qkv / bias rows go out before any tile, its table rows as soon as the
//     position returns and before the tiles, so q is ready about when the first tiles land.
//   * A unit's k / v / q writes go out after its last step (at its first step, in the middle of the tile
//     requests, they cost ~0.45 us per layer at the peak load).
//   * A finished unit is only parked (each wave's m, l, O in LDS); after every second unit and after the last
//     the workgroup waits for its slowest wave and all four waves merge the parked units, a slice of the
//     outputs each, with the hardware reciprocal for the division. Merging each unit as it finished, on the
//     last wave to arrive, cost ~0.7 us per layer more (the merging wave falls behind, the last merge runs
//     on one wave).
//   * Nothing is requested past the last tile (the pipeline's last two steps issue no load).
//   * K and V tiles go into LDS by non-temporal DMA; a step refills its K buffer as soon as the K operands are
//     in registers and its V buffer after the P.V operand reads.
// Measured at 192 rows x 2048 keys, 24 layers in a graph: 31.4 us per layer unfused and 32.4 fused (store
// included). Tried and slower: four tiles in flight per wave (+1 us), the first tiles requested before the
// position (+0.9 to +2.3 us: the table rows then return behind them), the table rows read through the scalar
// cache after the first tiles (+1.8 us), K kept in registers with its refill after the score products (+0.8
// us), one unit per workgroup over all compute units (k_decode_unit at grid 384: +2 us).
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
  int rot;  // the unit's first step (units start at different offsets; see k_decode_rows)
  rsrc_t kr, vr;
};

}  // namespace

// Per-wave partial of a finished unit as parked in LDS: m[PR], l[PR] (row sum over the lane groups), then O in
// rows of kOb floats (q head r16 < PR of the group, 64 dims). PR = 8 serves groups of up to 8 q heads (the
// engine's 7) in half the space.
template <int PR>
constexpr int park_floats() { return 2 * PR + PR * kOb; }

template <int PR>
__device__ __forceinline__ void park_partial(float *r, const SoftmaxState &S, const TileLane &tl) {
  const float lsum = sum_over_groups(S.lsum);
  if (tl.g == 0 && tl.r16 < PR) {
    r[tl.r16] = S.m;
    r[PR + tl.r16] = lsum;
  }
  if (PR == 16 || tl.r16 < PR) lds_store_4x16(r + 2 * PR + tl.r16 * kOb + 4 * tl.g, S.o[0], S.o[1], S.o[2], S.o[3]);
}

// Merges the NW parked partials of each of cnt (<= 2) units and writes the units' outputs. Wave partial v of
// unit s is at rs + v * rstride (rs = r0 or r1). The items (unit, q head, 4 dims) are shared out over the NW
// waves (item w * 64 + lane, then + NW * 64), so every wave of the workgroup merges a slice. Arithmetic of
// k_decode_combine's merge with a running maximum taken over the NW partials at once, the division as a
// multiplication by the hardware reciprocal.
template <int NW, int PR>
__device__ __forceinline__ void merge_units(const float *r0, const float *r1, int rstride, int cnt, int row0, int kh0,
                                            int row1, int kh1, uint16_t *out, int64_t s_ob, int64_t s_oh, int group,
                                            float sl2, int w, int lane) {
  const int per = group * 16, total = cnt * per;
  for (int t = w * 64 + lane; t < total; t += NW * 64) {
    const bool second = t >= per;
    const int rem = second ? t - per : t;
    const int head = rem >> 4, d4 = (rem & 15) * 4;
    const float *rb = second ? r1 : r0;
    float mv[NW], lv[NW];
    f32x4 ov[NW];
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const float *rv = rb + v * rstride;
      mv[v] = rv[head];
      lv[v] = rv[PR + head];
      ov[v] = *reinterpret_cast<const f32x4 *>(rv + 2 * PR + head * kOb + d4);
    }
    float M = kNegInf;
#pragma unroll
    for (int v = 0; v < NW; ++v) M = fmaxf(M, mv[v]);
    f32x4 num = {0.f, 0.f, 0.f, 0.f};
    float den = 0.f;
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const float wt = (mv[v] == kNegInf) ? 0.f : fast_exp2((mv[v] - M) * sl2);
      num += wt * ov[v];
      den += wt * lv[v];
    }
    const float rd = __builtin_amdgcn_rcpf(den);
    const u32x2 res{pack_bf16x2(num[0] * rd, num[1] * rd), pack_bf16x2(num[2] * rd, num[3] * rd)};
    const int row = second ? row1 : row0, kh = second ? kh1 : kh0;
    st8(out + (int64_t)row * s_ob + (int64_t)(kh * group + head) * s_oh + d4, res);
  }
}

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
  // K and V tiles of the two pipeline buffers (each read waits for its tile's DMA with a counted vmcnt)
  __shared__ __attribute__((aligned(16))) uint16_t kb0[NW * kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t kb1[NW * kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t vb0[NW * kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t vb1[NW * kVTile];
  // per-wave m, l, O of finished units (8 q heads), parked until MB of them are merged together
  constexpr int MB = 2, PR = 8;
  constexpr int PF = park_floats<PR>();
  __shared__ __attribute__((aligned(16))) float mrg[MB][NW * PF];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x;
  const int U = b * nkv;
  const int nmine = ((int)blockIdx.x < U) ? (U - 1 - (int)blockIdx.x) / G + 1 : 0;
  if (nmine == 0) return;

  TileLane tl;
  tl.init(lane);
  KLdsLane kl;
  kl.init(lane);
  uint16_t *const vbw[2] = {vb0 + w * kVTile, vb1 + w * kVTile};
  uint16_t *const kbw[2] = {kb0 + w * kVTile, kb1 + w * kVTile};

  // ---- metadata, inputs and the tile sources of unit i (i >= nmine: empty ranges, nothing is read) ----
  const rsrc_t lens_r = make_rsrc(lens, (uint32_t)b * 4u);
  const rsrc_t map_r = make_rsrc(rowmap, rowmap ? (uint32_t)b * 4u : 0u);
  const rsrc_t pos_r = make_rsrc(si.pos, FUSED ? (uint32_t)b * 4u : 0u);
  const rsrc_t slot_r = make_rsrc(si.slot, FUSED ? (uint32_t)b * 4u : 0u);
  auto unit_of = [&](int i) { return (int)blockIdx.x + i * G; };
  // wave w: tiles w, w + NW, ... of the unit, starting at step rot
  auto tile_of = [&](int rot, int j) { return w + NW * ((j + rot) & (SPW - 1)); };
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
    un.rot = u & (SPW - 1);
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
  RowUnit cur, nxt;
  u32x4 qc0, qc1, qn0, qn1;
  KVPatch ptc, ptn;
  ptc.col = -1;
  ptn.col = -1;
  QkvRaw rn;      // fused: raw chunks of the next unit, between its request and its rotation
  StoreDst sdc, sdn;  // fused: where the current / next unit's k / v / q go
  int mcur_p = 0, mcur_s = 0;  // fused: position / slot of unit i + 1 while it is prepared

  // ---- unit finish: park the wave's partial; every MB units (and after the last) the workgroup waits for its
  // slowest wave and all waves merge the parked units together, a slice each ----
  int nfin = 0, prow0 = 0, pkh0 = 0;
  auto finish = [&](const RowUnit &un) {
    const int n = nfin++;
    const int slot = n % MB;
    park_partial<PR>(mrg[slot] + w * PF, S, tl);
    S.reset();
    if (slot == 0) {
      prow0 = un.row;
      pkh0 = un.kh;
    }
    if (slot == MB - 1 || n == nmine - 1) {
      lds_barrier();  // every wave has parked (loads of the next unit stay in flight)
      merge_units<NW, PR>(mrg[0], mrg[1], PF, slot + 1, prow0, pkh0, un.row, un.kh, out, s_ob, s_oh, group, sl2,
                          w, lane);
      if (n < nmine - 1) lds_barrier();  // the area is read before the next unit parks into it
    }
  };

  // ---- steps: compute tile j of the current unit from buffer j % D, then request into it tile j + D of the
  // unit, or tile j + D - SPW of the next (one load sequence, sources selected) ----
  static_assert(D == 2, "wait counts assume one tile requested between a tile and its reads");
  // K(j+2) goes out as soon as tile j's K operands are in registers and V(j+2) after its P.V operand reads
  // (refilling each buffer at once, as one load sequence after the step, measured 0.2 us per layer slower at
  // the peak load, fused). Issued after V(j) when its reads wait: K(j+1), V(j+1) (unless `tail`) and K(j+2)
  // (when reloading); after K(j): V(j), then K(j+1), V(j+1) (unless `tail`).
  auto step = [&](uint16_t *xk, uint16_t *xv, int j, bool reload, bool tail) __attribute__((always_inline)) {
    const int t0 = 64 * tile_of(cur.rot, j);
    const bool in_cur = j + D < SPW;
    const rsrc_t kr = in_cur ? cur.kr : nxt.kr, vr = in_cur ? cur.vr : nxt.vr;
    const int tt = in_cur ? tile_of(cur.rot, j + D) : tile_of(nxt.rot, j + D - SPW);
    KTile X[1];
    if (t0 < cur.hi) {
      if (tail)
        read_k_tile<0>(X[0], xk, kl);
      else
        read_k_tile<16>(X[0], xk, kl);
    }
    if (reload) load_k_lds(xk, kr, (uint32_t)(64 * tt), kl);
    if (t0 < cur.hi) {
      if (reload)
        compute_step<1, 24, FUSED>(X, xv, t0, cur.hi, qc0, qc1, sl2, S, tl, lane, &ptc);
      else if (!tail)
        compute_step<1, 16, FUSED>(X, xv, t0, cur.hi, qc0, qc1, sl2, S, tl, lane, &ptc);
      else
        compute_step<1, 0, FUSED>(X, xv, t0, cur.hi, qc0, qc1, sl2, S, tl, lane, &ptc);
    }
    if (reload) load_v_lds(xv, vr, (uint32_t)(64 * tt), tl);
  };
  auto step_k = [&](int j, bool reload, bool tail) __attribute__((always_inline)) {
    step(kbw[j & 1], vbw[j & 1], j, reload, tail);
  };
  auto first_load = [&](int j) __attribute__((always_inline)) {
    load_tile_kv(kbw[j & 1], vbw[j & 1], cur.kr, cur.vr, (uint32_t)(64 * tile_of(cur.rot, j)), tl, kl);
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
      // position, and slower again with the table rows read through the scalar cache); the range is exact
      load_xb(u0, true, r0);
      load_tab(true, __builtin_amdgcn_readfirstlane(m0.praw), r0);
      resolve(0, m0, cur, true);
      first_load(0);
      // unit 0's rotation, once its table rows are in
      rope_unit(cur, true, __builtin_amdgcn_readfirstlane(m0.praw), __builtin_amdgcn_readfirstlane(m0.sraw), r0, qc0,
                qc1, ptc, sdc);
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
      step_k(j, true, false);
      if (FUSED && j == kRopeStep) rope_unit(nxt, true, mcur_p, mcur_s, rn, qn0, qn1, ptn, sdn);
    }
    // the unit's k / v / q go out after its last step (stored at its first step they cost ~0.45 us per layer at
    // the peak load); no row of the launch reads them back
    if (FUSED) rope_store(ptc, sdc);
    finish(cur);
    cur = nxt;
    qc0 = qn0;
    qc1 = qn1;
    if (FUSED) {
      ptc = ptn;
      sdc = sdn;
    }
  }
  // ---- the last unit: no request past its last tile ----
#pragma unroll
  for (int j = 0; j < SPW; ++j) step_k(j, j + D < SPW, j + 1 == SPW);
  if (FUSED) rope_store(ptc, sdc);
  finish(cur);
  // tiles past a unit's length are requested but not read: let every DMA land before the wave ends
  wait_vmcnt<0>();
}

// One unit (row, kv head) per workgroup: the launch for grids of at least one workgroup per unit (short rows,
// and row counts whose units do not fill the compute units twice over). Every unit streams at once. The work per
// wave, the order of its tiles (rotated as in k_decode_rows) and the merge are those of k_decode_rows, so the
// results are the same bits; each wave parks its partial in its first V buffer (free by then) and the four waves
// merge a slice of the outputs each. LDS: two K and two V tiles per wave, 128 KB, one workgroup per compute unit.
// Measured on MI355X at 64-256 units and no faster: 8 waves with K in registers (+2.5 us at 128 units), three
// or four tiles in flight per wave with K in registers (+2.5 / +2.9 us).
template <bool FUSED, int SPW>
__global__ __launch_bounds__(64 * kRowsNW, 2) void k_decode_unit(
    const uint16_t *__restrict__ q, int64_t s_qb, int64_t s_qh,
    uint16_t *kc, uint16_t *vc, int64_t s_kb, int64_t s_kh,
    int cache_rows, int cache_len, const int32_t *__restrict__ lens, const int32_t *__restrict__ rowmap,
    uint16_t *__restrict__ out, int64_t s_ob, int64_t s_oh, int b, int nq, int nkv, int group,
    float sl2, StoreIn si) {
  constexpr int NW = kRowsNW;
  constexpr int D = 2;  // tiles in flight per wave
  warm_kernargs<232>();
  static_assert(SPW % D == 0 && SPW >= 4, "steps per unit");
  __shared__ __attribute__((aligned(16))) uint16_t kb0[NW * kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t kb1[NW * kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t vb0[NW * kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t vb1[NW * kVTile];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int u = blockIdx.x;
  if (u >= b * nkv) return;
  const int row = u / nkv, kh = u - row * nkv;

  TileLane tl;
  tl.init(lane);
  KLdsLane kl;
  kl.init(lane);
  uint16_t *const vbw[2] = {vb0 + w * kVTile, vb1 + w * kVTile};
  uint16_t *const kbw[2] = {kb0 + w * kVTile, kb1 + w * kVTile};

  // ---- metadata: row map, length, position, slot (vector loads, in order with the tiles) ----
  const rsrc_t lens_r = make_rsrc(lens, (uint32_t)b * 4u);
  const rsrc_t map_r = make_rsrc(rowmap, rowmap ? (uint32_t)b * 4u : 0u);
  const rsrc_t pos_r = make_rsrc(si.pos, FUSED ? (uint32_t)b * 4u : 0u);
  const rsrc_t slot_r = make_rsrc(si.slot, FUSED ? (uint32_t)b * 4u : 0u);
  const uint32_t mo = (uint32_t)row * 4u;
  const int craw = bld4(map_r, mo);
  const int lraw = bld4(lens_r, mo);
  const int praw = FUSED ? bld4(pos_r, mo) : 0;
  const int sraw = FUSED ? bld4(slot_r, mo) : 0;

  int crow = -1, hi = 0;
  rsrc_t kr, vr;
  // exact = false: the range is the whole cache row (the length is not waited for; hi is set later)
  auto resolve = [&](bool exact) {
    int c = row;
    if (rowmap) c = __builtin_amdgcn_readfirstlane(craw);
    const bool ok = c >= 0 && c < cache_rows;
    crow = ok ? c : -1;
    hi = (ok && exact) ? min(max(__builtin_amdgcn_readfirstlane(lraw), 0), cache_len) : 0;
    const int64_t cb = (int64_t)(ok ? c : 0) * s_kb + (int64_t)kh * s_kh;
    const uint32_t bound = ok ? (uint32_t)(exact ? hi : cache_len) * kRow : 0u;
    kr = make_rsrc_wave(kc + cb, bound);
    vr = make_rsrc_wave(vc + cb, bound);
  };
  // wave w: tiles w, w + NW, ... of the unit, starting at step u % SPW (as k_decode_rows)
  const int rot = u & (SPW - 1);
  auto tile_of = [&](int j) { return w + NW * ((j + rot) & (SPW - 1)); };
  auto first_load = [&](int j) __attribute__((always_inline)) {
    load_tile_kv(kbw[j & 1], vbw[j & 1], kr, vr, (uint32_t)(64 * tile_of(j)), tl, kl);
  };

  u32x4 q0, q1;
  KVPatch pt;
  pt.col = -1;
  // fused: the k / v / q writes of bias_rope_store, from wave 0 (every lane of every wave issues them; the
  // range check drops the others')
  rsrc_t skr, svr, sqr;
  uint32_t sko = kOOR, svo = kOOR, sqo = kOOR;
  if (FUSED) {
    // qkv / bias chunks (lane head: fused_lane_head), then the position's table rows as soon as it returns,
    // ahead of every tile
    const int H = nq + 2 * nkv;
    const rsrc_t xr = make_rsrc_wave(si.qkv + (int64_t)row * si.s_qkv, (uint32_t)H * 128u);
    const rsrc_t br = make_rsrc(si.bias, si.bias ? (uint32_t)H * 128u : 0u);
    const uint32_t ho = (uint32_t)fused_lane_head(tl.r16, kh, group, nq, nkv) * 128u + 16u * tl.g;
    QkvRaw r;
    r.w[0] = bld16(xr, ho);
    r.w[1] = bld16(xr, ho + 64u);
    r.bb[0] = bld16(br, ho);
    r.bb[1] = bld16(br, ho + 64u);
    const int p = __builtin_amdgcn_readfirstlane(praw);
    const bool pv = p >= 0 && p < si.n_tab;
    const rsrc_t cr = make_rsrc_wave(si.cos_tab + (int64_t)(pv ? p : 0) * si.s_cs, pv ? 128u : 0u);
    const rsrc_t sr = make_rsrc_wave(si.sin_tab + (int64_t)(pv ? p : 0) * si.s_cs, pv ? 128u : 0u);
    const uint32_t og = 16u * tl.g;
    r.cs[0] = bld16(cr, og);
    r.cs[1] = bld16(cr, og + 64u);
    r.sn[0] = bld16(sr, og);
    r.sn[1] = bld16(sr, og + 64u);
    resolve(true);
    first_load(0);
    // the rotation (rope.h arithmetic), once the table rows are in
    const int srow = __builtin_amdgcn_readfirstlane(sraw);
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
    pt.col = (store_ok && srow == crow) ? sidx : -1;
    const bool w0 = w == 0;
    const int64_t kvo = (int64_t)(store_ok ? srow : 0) * s_kb + (int64_t)kh * s_kh + (int64_t)sidx * 64;
    skr = make_rsrc_wave(kc + kvo, store_ok ? 128u : 0u);
    svr = make_rsrc_wave(vc + kvo, store_ok ? 128u : 0u);
    const bool qw = si.qo != nullptr && pv;
    sqr = make_rsrc_wave(si.qo + (int64_t)(qw ? row : 0) * si.s_qo_r + (int64_t)kh * group * si.s_qo_h,
                         qw ? (uint32_t)((group - 1) * si.s_qo_h * 2 + 128) : 0u);
    sko = (w0 && klane) ? og : kOOR;
    svo = (w0 && vlane) ? og : kOOR;
    sqo = (w0 && tl.r16 < group) ? (uint32_t)(tl.r16 * si.s_qo_h * 2) + og : kOOR;
#pragma unroll
    for (int j = 1; j < D; ++j) first_load(j);
  } else {
    // unfused: the first tiles go out over the whole cache row before the length returns; the range is
    // narrowed after them
    const rsrc_t qr = make_rsrc(q + (int64_t)row * s_qb + (int64_t)kh * group * s_qh, (uint32_t)(group * s_qh * 2));
    const uint32_t qo = (uint32_t)(tl.r16 * s_qh * 2) + 16u * tl.g;
    q0 = bld16(qr, qo);
    q1 = bld16(qr, qo + 64u);
    resolve(false);
#pragma unroll
    for (int j = 0; j < D; ++j) first_load(j);
    resolve(true);
  }

  SoftmaxState S;
  S.reset();
  // tile j + 1 was requested after tile j, except for the last (wait counts as in k_decode_rows)
  static_assert(D == 2, "wait counts assume one tile requested after the one read");
  auto step = [&](uint16_t *xk, uint16_t *xv, int j) __attribute__((always_inline)) {
    const int t0 = 64 * tile_of(j);
    if (t0 < hi) {
      KTile X[1];
      if (j + 1 == SPW) {
        read_k_tile<0>(X[0], xk, kl);
        compute_step<1, 0, FUSED>(X, xv, t0, hi, q0, q1, sl2, S, tl, lane, &pt);
      } else {
        read_k_tile<16>(X[0], xk, kl);
        compute_step<1, 16, FUSED>(X, xv, t0, hi, q0, q1, sl2, S, tl, lane, &pt);
      }
    }
    if (j + D < SPW) load_tile_kv(xk, xv, kr, vr, (uint32_t)(64 * tile_of(j + D)), tl, kl);
  };
#pragma unroll
  for (int j = 0; j < SPW; ++j) step(kbw[j & 1], vbw[j & 1], j);
  if (FUSED) {  // the unit's k / v / q, after its last step (as k_decode_rows)
    bst16(skr, sko, pt.lo);
    bst16(skr, sko + 64u, pt.hi);
    bst16(svr, svo, pt.lo);
    bst16(svr, svo + 64u, pt.hi);
    bst16(sqr, sqo, pt.lo);
    bst16(sqr, sqo + 64u, pt.hi);
  }

  // ---- park (m, l, O) in this wave's first V buffer (free once every DMA has landed: tiles past the length
  // are requested but not read); the four waves merge a slice each ----
  wait_vmcnt<0>();
  park_partial<16>(reinterpret_cast<float *>(vbw[0]), S, tl);
  lds_barrier();
  merge_units<NW, 16>(reinterpret_cast<const float *>(vb0), nullptr, kVTile / 2, 1, row, kh, 0, 0, out, s_ob, s_oh,
                      group, sl2, w, lane);
}

template <bool FUSED, int SPW>
static void launch_rows(int grid, hipStream_t st, const uint16_t *q, int64_t s_qb, int64_t s_qh, uint16_t *kc,
                        uint16_t *vc, int64_t s_kb, int64_t s_kh, int cache_rows, int cache_len, const int32_t *lens,
                        const int32_t *rowmap, uint16_t *out, int64_t s_ob, int64_t s_oh, int b, int nq, int nkv,
                        int group, float sl2, const StoreIn &si) {
  if (grid >= b * nkv)  // one unit per workgroup
    hipLaunchKernelGGL((k_decode_unit<FUSED, SPW>), dim3(b * nkv), dim3(64 * kRowsNW), 0, st, q, s_qb, s_qh, kc, vc,
                       s_kb, s_kh, cache_rows, cache_len, lens, rowmap, out, s_ob, s_oh, b, nq, nkv, group, sl2, si);
  else
    hipLaunchKernelGGL((k_decode_rows<FUSED, SPW>), dim3(grid), dim3(64 * kRowsNW), 0, st, q, s_qb, s_qh, kc, vc,
                       s_kb, s_kh, cache_rows, cache_len, lens, rowmap, out, s_ob, s_oh, b, nq, nkv, group, sl2, si);
}

// Launches k_decode_rows when it serves the shape (whole rows per chunk at 4 waves x 1 tile per step, at
// most 16 steps per unit); returns false otherwise. Arguments are checked by the caller.
bool rows_launch(int grid, hipStream_t st, const uint16_t *q, int64_t s_qb, int64_t s_qh, uint16_t *kc, uint16_t *vc,
                 int64_t s_kb, int64_t s_kh, int cache_rows, int cache_len, const int32_t *lens, const int32_t *rowmap,
                 uint16_t *out, int64_t s_ob, int64_t s_oh, int b, int nq, int nkv, int group, float sl2,
                 const StoreIn &si) {
  const bool fused = si.qkv != nullptr;
  if (grid < b * nkv && group > 8) return false;  // k_decode_rows parks 8 q heads per wave
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
