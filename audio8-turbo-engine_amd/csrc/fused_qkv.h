// The store half of a fused store + decode launch, per (row, kv head) and per wave: the qkv / bias /
// RoPE-table chunks a wave needs (one head per lane), and from them, with the store kernel's arithmetic
// (rope.h), the Q^T operands of the decode, the new k / v column for the tile that holds it, and the
// cache / q writes of bias_rope_store (serve/fast_kernels.py:139-187).
//
// Lane roles (lane = 16 g + r16): r16 < group computes q head kh * group + r16, r16 == kLaneK the k
// head, r16 == kLaneV the v head; each lane holds dims 8g..8g+7 and 32+8g.. of its head.
#pragma once

#include "decode_tile.h"
#include "rope.h"

namespace a8 {

struct QkvRaw {
  u32x4 w[2], bb[2], cs[2], sn[2];
};

__device__ __forceinline__ int fused_lane_head(int r16, int kh, int group, int nq, int nkv) {
  return r16 < group ? kh * group + r16 : r16 == kLaneK ? nq + kh : r16 == kLaneV ? nq + nkv + kh : 0;
}

// Requests the lane's chunks of qkv row `row` (+ bias) and of table row p. A row that is not live reads
// nothing, a position outside the tables reads no table row (zeros).
__device__ __forceinline__ void load_qkv_raw(const StoreIn &si, bool live, int row, int kh, int p, int group,
                                             int nq, int nkv, const TileLane &tl, QkvRaw &r) {
  const int H = nq + 2 * nkv;
  const bool pv = live && p >= 0 && p < si.n_tab;
  const rsrc_t xr = make_rsrc_wave(si.qkv + (int64_t)(live ? row : 0) * si.s_qkv, live ? (uint32_t)H * 128u : 0u);
  const rsrc_t br = make_rsrc(si.bias, si.bias ? (uint32_t)H * 128u : 0u);
  const rsrc_t cr = make_rsrc_wave(si.cos_tab + (int64_t)(pv ? p : 0) * si.s_cs, pv ? 128u : 0u);
  const rsrc_t sr = make_rsrc_wave(si.sin_tab + (int64_t)(pv ? p : 0) * si.s_cs, pv ? 128u : 0u);
  const uint32_t og = 16u * tl.g, ho = (uint32_t)fused_lane_head(tl.r16, kh, group, nq, nkv) * 128u + og;
  r.w[0] = bld16(xr, ho);
  r.w[1] = bld16(xr, ho + 64u);
  r.bb[0] = bld16(br, ho);
  r.bb[1] = bld16(br, ho + 64u);
  r.cs[0] = bld16(cr, og);
  r.cs[1] = bld16(cr, og + 64u);
  r.sn[0] = bld16(sr, og);
  r.sn[1] = bld16(sr, og + 64u);
}

// One RoPE pass per lane over the chunks of load_qkv_raw. Gives the Q^T operands q0 / q1 (zero when the
// position is outside the tables: the reference reads no table row there) and the patch column (the new
// key, when the row stores into the cache row it attends, crow == srow). With `store`, lanes kLaneK /
// kLaneV write k / v to kc / vc[srow, kh, p % ring] and the q lanes write q to si.qo (when given).
__device__ __forceinline__ void apply_qkv_raw(const StoreIn &si, const QkvRaw &r, bool live, int row, int kh,
                                              int p, int srow, int crow, int cache_rows, int cache_len,
                                              int group, uint16_t *kc, uint16_t *vc, int64_t s_kb, int64_t s_kh,
                                              int64_t s_ks, bool store, const TileLane &tl, u32x4 &q0, u32x4 &q1,
                                              KVPatch &pt) {
  const bool pv = live && p >= 0 && p < si.n_tab;
  const int sidx = pv ? p % si.ring : 0;
  const bool store_ok = pv && srow >= 0 && srow < cache_rows && sidx < cache_len;
  float xl[8], xh[8], ol[8], oh[8];
  rope_x(r.w[0], r.w[1], r.bb[0], r.bb[1], si.bias != nullptr, xl, xh);
  rope_rotate_f(xl, xh, r.cs[0], r.cs[1], r.sn[0], r.sn[1], ol, oh);
  const bool vlane = tl.r16 == kLaneV;
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
  if (store) {
    uint16_t *dst = nullptr;
    if (store_ok && (tl.r16 == kLaneK || vlane))
      dst = (vlane ? vc : kc) + (int64_t)srow * s_kb + (int64_t)kh * s_kh + (int64_t)sidx * s_ks;
    else if (si.qo && qlive)
      dst = si.qo + (int64_t)row * si.s_qo_r + (int64_t)(kh * group + tl.r16) * si.s_qo_h;
    if (dst) {
      st16(dst + 8 * tl.g, pt.lo);
      st16(dst + 32 + 8 * tl.g, pt.hi);
    }
  }
}

}  // namespace a8
