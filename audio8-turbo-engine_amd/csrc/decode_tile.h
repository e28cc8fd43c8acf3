// One wavefront's 64-key decode tile: loads, S^T = K.Q^T, online softmax, O^T += V^T.P^T.
// Shared by the split/combine kernels (decode.hip) and the streaming kernel (decode_stream.hip).
//
// Layout (v_mfma_f32_16x16x32_bf16, lane l = 16g + r16):
//   * S^T tile (c, t) of a 64-key tile (c = 32-key chunk, t = 16-key half of it): A = K rows with
//     row r16 <-> key 32c + 8(r16/4) + 4t + r16%4, B = Q^T with column r16 <-> q head r16 of the
//     group (zero past the group). Its C layout, row 4g+i <-> key 32c + 8g + 4t + i, is directly the
//     P^T B operand of O^T += V^T . P^T (lane group g owns keys 8g..8g+7 of chunk c).
//   * V: lane (kg = l%8, dc = l/8) loads keys 8kg..8kg+7 x dims 8dc..8dc+7 (each load instruction
//     reads 8 whole 128-byte key rows), transposes 8x8 in registers with v_perm and stores V^T[d][key]
//     into a wave-private LDS tile; the V^T A operand is then one 128-bit LDS read.
//   * Softmax state per lane (column r16 = q head): running max m in raw score units, the lane
//     group's partial row sum, O^T rows d = 16dt + 4g + i. exp2((s - m) * scale * log2 e) is one FMA
//     and one v_exp; the accumulator rescale is skipped when no column's max moved.
#pragma once

#include "a8_common.h"

namespace a8 {

constexpr int kVRow = 72;      // LDS row of a transposed V tile: 64 keys + 8 pad (144 B, 16-B aligned)
constexpr uint32_t kRow = 128;  // bytes per cached key row (head_dim 64 bf16, rows contiguous)
// Row stride (floats) of the per-wave O partials merged through LDS: 64 dims + 4, so the 16 rows a
// wave writes at once start in different banks.
constexpr int kOb = 68;

struct KVTile {
  u32x4 ka[2][2][2];  // [c][t][dim half]
  u32x4 vr[8];        // V rows 8kg + j, dims 8dc..8dc+7
};

// Per-lane byte offsets inside a tile. The (c, t, half) and j steps are compile-time constants, so
// each load is one base register plus an immediate offset: K rows of chunk c = 1 start 4096 B in, past
// the 12-bit immediate, hence a second K base.
struct TileLane {
  int r16, g, kg, dc;
  uint32_t kb0, kb1;  // K: rows 8(r16/4) + r16%4 (+32 for kb1), dims 8g..
  uint32_t vb;        // V: rows 8kg, dims 8dc..
  __device__ __forceinline__ void init(int lane) {
    r16 = lane & 15;
    g = lane >> 4;
    kg = lane & 7;  // lanes 0-7 hold consecutive key blocks of one dim block: their V^T rows are one
    dc = lane >> 3; // contiguous 128 B run in LDS, so the V^T writes are free of bank conflicts
    kb0 = (uint32_t)(8 * (r16 >> 2) + (r16 & 3)) * kRow + 16u * g;
    kb1 = kb0 + 32u * kRow;
    vb = (uint32_t)(8 * kg) * kRow + 16u * dc;
  }
};

// Loads keys [t0, t0+64) of one (cache row, kv head): kr / vr are buffers whose range ends at the
// last valid key (rows past it read as zeros, without memory traffic).
__device__ __forceinline__ void load_tile(KVTile &T, rsrc_t kr, rsrc_t vr, uint32_t t0, const TileLane &L) {
  const uint32_t base = t0 * kRow;
  const uint32_t k0 = base + L.kb0, k1 = base + L.kb1, v0 = base + L.vb;
  T.ka[0][0][0] = bld16(kr, k0);
  T.ka[0][0][1] = bld16(kr, k0 + 64u);
  T.ka[0][1][0] = bld16(kr, k0 + 4u * kRow);
  T.ka[0][1][1] = bld16(kr, k0 + 4u * kRow + 64u);
  T.ka[1][0][0] = bld16(kr, k1);
  T.ka[1][0][1] = bld16(kr, k1 + 64u);
  T.ka[1][1][0] = bld16(kr, k1 + 4u * kRow);
  T.ka[1][1][1] = bld16(kr, k1 + 4u * kRow + 64u);
#pragma unroll
  for (int j = 0; j < 8; ++j) T.vr[j] = bld16(vr, v0 + (uint32_t)j * kRow);
}

struct SoftmaxState {
  float m;     // running max of the raw scores q.k (-inf before the first key)
  float lsum;  // this lane group's share of the row sum, relative to m
  f32x4 o[4];  // O^T rows 16dt + 4g + i (this lane's column)
  __device__ __forceinline__ void reset() {
    m = kNegInf;
    lsum = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
};

// bf16 8x8 transpose: out[c] = element c of in[0..7]; dword e of out[c] pairs rows 2e and 2e+1.
__device__ __forceinline__ void transpose8x8(const u32x4 (&in)[8], u32x4 (&out)[8]) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int e = 0; e < 4; ++e) out[c][e] = __builtin_amdgcn_perm(in[2 * e + 1][c >> 1], in[2 * e][c >> 1], sel);
  }
}

// S^T for the tile (raw scores), with keys >= hi set to -inf when MASK.
template <bool MASK>
__device__ __forceinline__ float tile_scores(const KVTile &T, int t0, int hi, u32x4 qB0, u32x4 qB1,
                                             f32x4 (&s)[2][2], const TileLane &L) {
  float mt = kNegInf;
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4 a = mfma16x16x32(T.ka[c][t][0], qB0, f32x4{0.f, 0.f, 0.f, 0.f});
      a = mfma16x16x32(T.ka[c][t][1], qB1, a);
      if (MASK) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (t0 + 32 * c + 8 * L.g + 4 * t + i >= hi) a[i] = kNegInf;
      }
      mt = fmaxf(mt, fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3])));
      s[c][t] = a;
    }
  return mt;
}

// Loads keys [t0, t0 + 64 NT) as NT tiles.
template <int NT>
__device__ __forceinline__ void load_step(KVTile (&T)[NT], rsrc_t kr, rsrc_t vr, uint32_t t0, const TileLane &L) {
#pragma unroll
  for (int h = 0; h < NT; ++h) load_tile(T[h], kr, vr, t0 + 64u * h, L);
}

// Consumes keys [t0, min(t0 + 64 NT, hi)) of the NT tiles T (t0 < hi); rows past hi may hold anything
// (their scores are masked and their values zeroed). One softmax update covers all NT tiles, so with
// NT = 2 the MFMA, exp and max chains of two tiles run side by side and the cross-lane reductions and
// the rescale happen once per 128 keys. qB0 / qB1: Q^T operands (dims 8g.. and 32+8g..).
// sl2 = scale * log2(e). vt: this wave's LDS V^T tiles (NT x 64 rows of kVRow).
template <int NT>
__device__ __forceinline__ void compute_step(const KVTile (&T)[NT], int t0, int hi, u32x4 qB0, u32x4 qB1, float sl2,
                                             SoftmaxState &S, uint16_t *vt, const TileLane &L) {
  f32x4 s[NT][2][2];
  const bool full = t0 + 64 * NT <= hi;
  float mt = kNegInf;
  if (full) {
#pragma unroll
    for (int h = 0; h < NT; ++h) mt = fmaxf(mt, tile_scores<false>(T[h], t0 + 64 * h, hi, qB0, qB1, s[h], L));
  } else {
#pragma unroll
    for (int h = 0; h < NT; ++h) mt = fmaxf(mt, tile_scores<true>(T[h], t0 + 64 * h, hi, qB0, qB1, s[h], L));
  }
  // V^T of each tile into its LDS slot; value rows past the range count as zeros, as masked loads
  // would read them
#pragma unroll
  for (int h = 0; h < NT; ++h) {
    u32x4 vtr[8];
    if (full) {
      transpose8x8(T[h].vr, vtr);
    } else {
      u32x4 vz[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) vz[j] = (t0 + 64 * h + 8 * L.kg + j < hi) ? T[h].vr[j] : u32x4{0u, 0u, 0u, 0u};
      transpose8x8(vz, vtr);
    }
#pragma unroll
    for (int dd = 0; dd < 8; ++dd) st16(vt + (64 * h + 8 * L.dc + dd) * kVRow + 8 * L.kg, vtr[dd]);
  }
  mt = max_over_groups(mt);
  const float mn = fmaxf(S.m, mt);
  const float mc = mn * sl2;
  const float alpha = (S.m == kNegInf) ? 0.f : fast_exp2(__builtin_fmaf(S.m, sl2, -mc));
  float ps = 0.f;
  u32x4 pB[NT][2];
#pragma unroll
  for (int h = 0; h < NT; ++h)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[i] = fast_exp2(__builtin_fmaf(s[h][c][t][i], sl2, -mc));
          ps += p[i];
        }
        pB[h][c][2 * t] = pack_bf16x2(p[0], p[1]);
        pB[h][c][2 * t + 1] = pack_bf16x2(p[2], p[3]);
      }
  S.lsum = S.lsum * alpha + ps;
  S.m = mn;

  wave_lds_fence();
  if (__ballot(alpha != 1.f)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) S.o[dt] *= alpha;
  }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
    for (int h = 0; h < NT; ++h)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const u32x4 vA = ld16(vt + (64 * h + 16 * dt + L.r16) * kVRow + 32 * c + 8 * L.g);
        S.o[dt] = mfma16x16x32(vA, pB[h][c], S.o[dt]);
      }
  }
  wave_lds_fence();
}

// One 64-key tile (compute_step with NT = 1).
__device__ __forceinline__ void compute_tile(const KVTile &T, int t0, int hi, u32x4 qB0, u32x4 qB1, float sl2,
                                             SoftmaxState &S, uint16_t *vt, const TileLane &L) {
  compute_step<1>(reinterpret_cast<const KVTile(&)[1]>(T), t0, hi, qB0, qB1, sl2, S, vt, L);
}

}  // namespace a8
