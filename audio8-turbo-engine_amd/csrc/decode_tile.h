// One wavefront's decode step over 64 NT keys: loads, S^T = K.Q^T, online softmax, O^T += V^T.P^T.
// Shared by the split/combine kernels (decode.hip) and the streaming kernel (decode_stream.hip).
//
// Layout (v_mfma_f32_16x16x32_bf16, lane l = 16g + r16):
//   * S^T tile (c, t) of a 64-key tile (c = 32-key chunk, t = 16-key half of it): A = K rows with
//     row r16 <-> key 32c + 8(r16/4) + 4t + r16%4, B = Q^T with column r16 <-> q head r16 of the
//     group (zero past the group). Its C layout, row 4g+i <-> key 32c + 8g + 4t + i, is directly the
//     P^T B operand of O^T += V^T . P^T (lane group g owns keys 8g..8g+7 of chunk c). K goes from
//     memory into registers.
//   * V goes from memory straight into a wave-private LDS tile (buffer_load ... lds, 8 instructions
//     of 8 whole 128-byte key rows each), row-major with the 16-byte chunks of row r permuted by
//     chunk ^= 2 * ((r & 3) ^ ((r >> 3) & 1)). The V^T A operand (dims 16dt + r16, keys 32c + 8g..+7)
//     is two transposing LDS reads (ds_read_b64_tr_b16, 4 keys each); the permutation spreads each
//     read's 4 rows x 32 bytes, and the two row blocks served together, over distinct banks.
//   * Softmax state per lane (column r16 = q head): running max m in raw score units, the lane
//     group's partial row sum, O^T rows d = 16dt + 4g + i. exp2((s - m) * scale * log2 e) is one FMA
//     and one v_exp; the accumulator rescale is skipped when no column's max moved.
#pragma once

#include "a8_common.h"

namespace a8 {

constexpr uint32_t kRow = 128;   // bytes per cached key row (head_dim 64 bf16, rows contiguous)
constexpr int kVTile = 64 * 64;  // bf16 elements of one V tile in LDS (8 KB)
// Row stride (floats) of the per-wave O partials merged through LDS: 64 dims + 4, so the 16 rows a
// wave writes at once start in different banks.
constexpr int kOb = 68;

struct KTile {
  u32x4 ka[2][2][2];  // [c][t][dim half]
};

// Per-lane offsets, computed once. K: one base register plus immediate offsets per load (rows of
// chunk c = 1 start 4096 B in, past the 12-bit immediate, hence a second base). V DMA: the load of
// rows 8j..8j+7 (j = 0..7) uses vd[j & 1] (the chunk permutation alternates with row bit 3). V^T
// reads: vt[dt] for dim block dt; the (c, half) steps are immediates.
struct TileLane {
  int r16, g;
  uint32_t kb0, kb1;  // K: rows 8(r16/4) + r16%4 (+32 for kb1), dims 8g..
  uint32_t vd[2];     // V DMA source offset inside a tile (row l/8 of the 8-row block, permuted chunk)
  uint32_t vt[4];     // V^T read: LDS byte offset inside a tile for dim block dt
  __device__ __forceinline__ void init(int lane) {
    r16 = lane & 15;
    g = lane >> 4;
    kb0 = (uint32_t)(8 * (r16 >> 2) + (r16 & 3)) * kRow + 16u * g;
    kb1 = kb0 + 32u * kRow;
    const int row8 = lane >> 3, ch = lane & 7;
#pragma unroll
    for (int p = 0; p < 2; ++p) vd[p] = (uint32_t)row8 * kRow + 16u * (uint32_t)(ch ^ (2 * ((row8 & 3) ^ p)));
    // lane reads row 32c + 8g + 4e + r16/4, dims 16dt + 4(r16%4)..: chunk 2dt + (r16/2)%2, half r16%2
    const int s = (r16 >> 2) ^ (g & 1);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      vt[dt] = (uint32_t)(8 * g + (r16 >> 2)) * kRow + 16u * ((r16 >> 1) & 1) + 8u * (r16 & 1) + 32u * (dt ^ s);
  }
};

// Cache policy of the V tile DMA: nt (non-temporal). Each V row is read once, as whole 128-byte lines, so
// nothing is lost by not keeping it; streamed without it, the peak-load decode (192 x 2048, fused store) took
// 36.1 us per layer on MI355X, with it 33.6. The K loads keep the default policy: each 128-byte row is read as
// two 64-byte halves by two instructions, and non-temporal K loads measured slower (37.3 us), the second
// half finding its line gone.
#ifndef A8_TILE_CPOL_V
#define A8_TILE_CPOL_V 2
#endif
// Loads keys [t0, t0+64) of one (cache row, kv head): K into T, V into the LDS tile vtile (8 KB,
// this wave's). kr / vr are buffers whose range ends at the last key they may read (rows past it read
// as zeros, without memory traffic).
__device__ __forceinline__ void load_tile(KTile &T, uint16_t *vtile, rsrc_t kr, rsrc_t vr, uint32_t t0,
                                          const TileLane &L) {
  // The DMA writes vtile whenever its data returns: every earlier LDS access of this wave (the reads
  // of the step that last used this buffer, zeroed rows) must have completed. s_waitcnt lgkmcnt(0),
  // vmcnt and expcnt left at their maxima.
  __builtin_amdgcn_s_waitcnt(0xC07F);
  const uint32_t base = t0 * kRow;
  const uint32_t k0 = base + L.kb0, k1 = base + L.kb1;
  T.ka[0][0][0] = bld16(kr, k0);
  T.ka[0][0][1] = bld16(kr, k0 + 64u);
  T.ka[0][1][0] = bld16(kr, k0 + 4u * kRow);
  T.ka[0][1][1] = bld16(kr, k0 + 4u * kRow + 64u);
  T.ka[1][0][0] = bld16(kr, k1);
  T.ka[1][0][1] = bld16(kr, k1 + 64u);
  T.ka[1][1][0] = bld16(kr, k1 + 4u * kRow);
  T.ka[1][1][1] = bld16(kr, k1 + 4u * kRow + 64u);
  // rows 8j..8j+7 land at vtile + 1024 j: j < 4 through the immediate, j >= 4 from a base 4 KB on
  const uint32_t v0 = base + L.vd[0], v1 = base + L.vd[1];
  char *lo = reinterpret_cast<char *>(vtile), *hi = lo + 4096;
  bld16_lds<0, A8_TILE_CPOL_V>(vr, lo, v0, 0u);
  bld16_lds<1024, A8_TILE_CPOL_V>(vr, lo, v1, 0u);
  bld16_lds<2048, A8_TILE_CPOL_V>(vr, lo, v0, 0u);
  bld16_lds<3072, A8_TILE_CPOL_V>(vr, lo, v1, 0u);
  bld16_lds<0, A8_TILE_CPOL_V>(vr, hi, v0, 4096u);
  bld16_lds<1024, A8_TILE_CPOL_V>(vr, hi, v1, 4096u);
  bld16_lds<2048, A8_TILE_CPOL_V>(vr, hi, v0, 4096u);
  bld16_lds<3072, A8_TILE_CPOL_V>(vr, hi, v1, 4096u);
}

// ---- K tiles in LDS (the whole-row decode kernels) ----
// K, like V, goes into a wave-private LDS tile by DMA, whole 128-byte rows (8 rows per instruction) with the
// non-temporal policy, and the A operands are read from there: the register loads of the S^T layout take each
// row as two 64-byte halves, and streamed that way K cost ~0.5 us per layer more at the peak load (the halves
// cannot be non-temporal). The 16-byte chunks of row r are permuted by chunk ^ kswz(r), so the 16 rows one
// A-operand read touches per lane group fall in 8 distinct 16-byte bank groups per 8 lanes.
__device__ __forceinline__ int kswz(int r) { return (r & 3) | (((r >> 3) & 1) << 2); }

struct KLdsLane {
  uint32_t kd[2];     // DMA source offset inside a tile for rows 8j + lane / 8: j even / odd (row bit 3)
  uint32_t ko0, ko1;  // A-operand reads: row 8(r16/4) + r16%4, chunk g (dims 8g..) and 4 + g (32 + 8g..)
  __device__ __forceinline__ void init(int lane) {
    const int row8 = lane >> 3, ch8 = lane & 7;
    kd[0] = (uint32_t)row8 * kRow + 16u * (uint32_t)(ch8 ^ (row8 & 3));
    kd[1] = (uint32_t)row8 * kRow + 16u * (uint32_t)(ch8 ^ ((row8 & 3) | 4));
    const int r16 = lane & 15, g = lane >> 4;
    const int krow = 8 * (r16 >> 2) + (r16 & 3), kz = kswz(krow);
    ko0 = (uint32_t)krow * kRow + 16u * (uint32_t)(g ^ kz);
    ko1 = (uint32_t)krow * kRow + 16u * (uint32_t)((4 + g) ^ kz);
  }
};

// The halves of load_tile_kv, for a step that refills its K buffer as soon as the K operands are in registers
// and its V buffer after the P.V operand reads: keys [t0, t0+64) into ktile / vtile (8 DMA instructions each).
__device__ __forceinline__ void load_k_lds(uint16_t *ktile, rsrc_t kr, uint32_t t0, const KLdsLane &K) {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's LDS reads of the buffer done (see load_tile)
  const uint32_t base = t0 * kRow;
  const uint32_t a0 = base + K.kd[0], a1 = base + K.kd[1];
  char *kl = reinterpret_cast<char *>(ktile), *kh = kl + 4096;
  bld16_lds<0, 2>(kr, kl, a0, 0u);
  bld16_lds<1024, 2>(kr, kl, a1, 0u);
  bld16_lds<2048, 2>(kr, kl, a0, 0u);
  bld16_lds<3072, 2>(kr, kl, a1, 0u);
  bld16_lds<0, 2>(kr, kh, a0, 4096u);
  bld16_lds<1024, 2>(kr, kh, a1, 4096u);
  bld16_lds<2048, 2>(kr, kh, a0, 4096u);
  bld16_lds<3072, 2>(kr, kh, a1, 4096u);
}
__device__ __forceinline__ void load_v_lds(uint16_t *vtile, rsrc_t vr, uint32_t t0, const TileLane &L) {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's LDS reads of the buffer done (see load_tile)
  const uint32_t base = t0 * kRow;
  const uint32_t v0 = base + L.vd[0], v1 = base + L.vd[1];
  char *lo = reinterpret_cast<char *>(vtile), *hi = lo + 4096;
  bld16_lds<0, 2>(vr, lo, v0, 0u);
  bld16_lds<1024, 2>(vr, lo, v1, 0u);
  bld16_lds<2048, 2>(vr, lo, v0, 0u);
  bld16_lds<3072, 2>(vr, lo, v1, 0u);
  bld16_lds<0, 2>(vr, hi, v0, 4096u);
  bld16_lds<1024, 2>(vr, hi, v1, 4096u);
  bld16_lds<2048, 2>(vr, hi, v0, 4096u);
  bld16_lds<3072, 2>(vr, hi, v1, 4096u);
}

// Loads keys [t0, t0+64) of one (cache row, kv head): K into the LDS tile ktile, V into vtile (8 KB each, this
// wave's), both non-temporal. Same range semantics as load_tile.
__device__ __forceinline__ void load_tile_kv(uint16_t *ktile, uint16_t *vtile, rsrc_t kr, rsrc_t vr, uint32_t t0,
                                             const TileLane &L, const KLdsLane &K) {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's LDS reads of the buffers done (see load_tile)
  const uint32_t base = t0 * kRow;
  const uint32_t a0 = base + K.kd[0], a1 = base + K.kd[1];
  char *kl = reinterpret_cast<char *>(ktile), *kh = kl + 4096;
  bld16_lds<0, 2>(kr, kl, a0, 0u);
  bld16_lds<1024, 2>(kr, kl, a1, 0u);
  bld16_lds<2048, 2>(kr, kl, a0, 0u);
  bld16_lds<3072, 2>(kr, kl, a1, 0u);
  bld16_lds<0, 2>(kr, kh, a0, 4096u);
  bld16_lds<1024, 2>(kr, kh, a1, 4096u);
  bld16_lds<2048, 2>(kr, kh, a0, 4096u);
  bld16_lds<3072, 2>(kr, kh, a1, 4096u);
  const uint32_t v0 = base + L.vd[0], v1 = base + L.vd[1];
  char *lo = reinterpret_cast<char *>(vtile), *hi = lo + 4096;
  bld16_lds<0, 2>(vr, lo, v0, 0u);
  bld16_lds<1024, 2>(vr, lo, v1, 0u);
  bld16_lds<2048, 2>(vr, lo, v0, 0u);
  bld16_lds<3072, 2>(vr, lo, v1, 0u);
  bld16_lds<0, 2>(vr, hi, v0, 4096u);
  bld16_lds<1024, 2>(vr, hi, v1, 4096u);
  bld16_lds<2048, 2>(vr, hi, v0, 4096u);
  bld16_lds<3072, 2>(vr, hi, v1, 4096u);
}

// The S^T A operands of a K tile in LDS (load_tile_kv's layout) into registers, as load_tile leaves them.
// VW: vector-memory operations this wave has certainly issued after the tile's load_tile_kv (the later
// tiles' requests; 16 per tile). Its K DMAs are the sequence's first 8, so they have landed at
// vmcnt(VW + 8).
template <int VW>
__device__ __forceinline__ void read_k_tile(KTile &T, const uint16_t *ktile, const KLdsLane &K) {
  wait_vmcnt<VW + 8>();
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const char *kp = reinterpret_cast<const char *>(ktile) + (32 * c + 4 * t) * kRow;
      T.ka[c][t][0] = lds_ld16(kp + K.ko0);
      T.ka[c][t][1] = lds_ld16(kp + K.ko1);
    }
}

// Loads keys [t0, t0 + 64 NT) as NT tiles (V tiles consecutive in vbuf).
template <int NT>
__device__ __forceinline__ void load_step(KTile (&T)[NT], uint16_t *vbuf, rsrc_t kr, rsrc_t vr, uint32_t t0,
                                          const TileLane &L) {
#pragma unroll
  for (int h = 0; h < NT; ++h) load_tile(T[h], vbuf + h * kVTile, kr, vr, t0 + 64u * h, L);
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

// S^T for the tile (raw scores), with keys >= hi set to -inf when MASK.
template <bool MASK>
__device__ __forceinline__ float tile_scores(const KTile &T, int t0, int hi, u32x4 qB0, u32x4 qB1,
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

// Zeroes the rows [from, 64) of an LDS V tile (whole rows: the chunk permutation does not matter).
__device__ __forceinline__ void zero_rows(uint16_t *vtile, int from, int lane) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int row = 8 * j + (lane >> 3);
    if (row >= from) st16(vtile + row * 64 + 8 * (lane & 7), u32x4{0u, 0u, 0u, 0u});
  }
}

// One key column whose K / V in the cache are being replaced in this launch (the fused store + decode):
// the tile holding it takes the new row from registers, whatever its loads returned. lo / hi are dims
// 8g.. and 32+8g.. of a lane's RoPE result: lane (r16 = kLaneK, g) holds the new k, lane (kLaneV, g) the
// new v. col < 0: no column.
constexpr int kLaneK = 14, kLaneV = 15;
struct KVPatch {
  int col;
  u32x4 lo, hi;
};

// Inputs of a fused store + decode launch (a8_store_decode_stream, a8_store_decode_flat): the
// bias_rope_store arguments the decode does not already take. Query row r stores into cache row slot[r]
// and attends cache row rowmap[r] (or r).
struct StoreIn {
  const int32_t *slot;
  const uint16_t *qkv;
  int64_t s_qkv;
  const uint16_t *bias;  // nullptr: no bias
  const uint16_t *cos_tab, *sin_tab;
  int64_t s_cs;
  int n_tab;
  const int32_t *pos;
  uint16_t *qo;  // nullptr: q is not written out
  int64_t s_qo_r, s_qo_h;
  int ring;
};

// Replaces key column pt.col (when it lies in [t0, t0 + 64 NT)) in the tiles. patch_k: its K row in the
// four lanes that hold it (ka[c][t][*] of lanes r16 = 4 (r / 8) + r % 4, r = column % 32; the k comes
// from lane kLaneK of the same group by a shuffle). patch_v: its V row in the LDS tile (chunks permuted
// as the DMA placed them, written by the kLaneV lanes), after the tile's DMA has landed.
template <int NT>
__device__ __forceinline__ void patch_k(KTile (&T)[NT], int t0, const KVPatch &pt, const TileLane &L) {
  const int kk = pt.col - t0;
  if (kk < 0 || kk >= 64 * NT) return;
  const int h = kk >> 6, r64 = kk & 63, cc = r64 >> 5, rr = r64 & 31;
  const int r16s = 4 * (rr >> 3) + (rr & 3), ts = (rr >> 2) & 1;
  const int src = 16 * L.g + kLaneK;
  u32x4 klo, khi;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    klo[e] = (uint32_t)__shfl((int)pt.lo[e], src);
    khi[e] = (uint32_t)__shfl((int)pt.hi[e], src);
  }
  const bool mine = L.r16 == r16s;
#pragma unroll
  for (int hh = 0; hh < NT; ++hh)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const bool sel = mine && hh == h && c == cc && t == ts;
        T[hh].ka[c][t][0] = sel ? klo : T[hh].ka[c][t][0];
        T[hh].ka[c][t][1] = sel ? khi : T[hh].ka[c][t][1];
      }
}
template <int NT>
__device__ __forceinline__ void patch_v(uint16_t *vbuf, int t0, const KVPatch &pt, const TileLane &L) {
  const int kk = pt.col - t0;
  if (kk < 0 || kk >= 64 * NT || L.r16 != kLaneV) return;
  const int h = kk >> 6, r64 = kk & 63;
  const int s = (r64 & 3) ^ ((r64 >> 3) & 1);
  uint16_t *row = vbuf + h * kVTile + r64 * 64;
  st16(row + 8 * (L.g ^ (2 * s)), pt.lo);
  st16(row + 8 * ((4 + L.g) ^ (2 * s)), pt.hi);
}

// Consumes keys [t0, min(t0 + 64 NT, hi)) of the NT tiles (K in T, V in vbuf; t0 < hi). Rows past hi
// may hold anything: their scores are masked and their LDS value rows zeroed (0 * NaN would not be
// 0). One softmax update covers all NT tiles. qB0 / qB1: Q^T operands (dims 8g.. and 32+8g..).
// sl2 = scale * log2(e). With PATCH, key column pt.col takes the new K / V row first.
// VW: vector-memory operations this wave has certainly issued after the last DMA of the V tiles (the next
// step's requests); every LDS access of the V tiles (patch, zeroed rows, operand reads) follows
// s_waitcnt vmcnt(VW).
template <int NT, int VW, bool PATCH = false>
__device__ __forceinline__ void compute_step(KTile (&T)[NT], uint16_t *vbuf, int t0, int hi, u32x4 qB0,
                                             u32x4 qB1, float sl2, SoftmaxState &S, const TileLane &L,
                                             int lane, const KVPatch *pt = nullptr) {
  if (PATCH) patch_k<NT>(T, t0, *pt, L);
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

  if (__ballot(alpha != 1.f)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) S.o[dt] *= alpha;
  }
  wait_vmcnt<VW>();  // the V tiles have landed
  if (PATCH) patch_v<NT>(vbuf, t0, *pt, L);
  if (!full) {
#pragma unroll
    for (int h = 0; h < NT; ++h) zero_rows(vbuf + h * kVTile, hi - (t0 + 64 * h), lane);
  }
#pragma unroll
  for (int h = 0; h < NT; ++h) {
    const char *vb = reinterpret_cast<const char *>(vbuf + h * kVTile);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const char *p = vb + L.vt[dt] + 32 * c * kRow;
        const u32x2 lo = lds_tr16(p), hi2 = lds_tr16(p + 4 * kRow);
        S.o[dt] = mfma16x16x32(u32x4{lo[0], lo[1], hi2[0], hi2[1]}, pB[h][c], S.o[dt]);
      }
  }
}

// ---- Partials exchanged between the workgroups of one launch (the in-kernel merges; kSC1) ----

// Called by a whole wave after its partial's stores: true in the wave that brings the count to `arrivals`,
// which also puts the counter back to 0 for the next launch (every arrival of this one is in).
__device__ __forceinline__ bool last_arrival(int32_t *ctr, int arrivals) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the partial has reached the coherent level
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  int old = 0;
  if (__lane_id() == 0) old = atomicAdd(ctr, 1);
  old = __shfl(old, 0);
  const bool last = old == arrivals - 1;
  if (last && __lane_id() == 0) *ctr = 0;
  return last;
}

// Merge of one (row, kv head)'s partials laid out [head][split] (acc 64 floats, ml 2 floats each), in
// split order with a running maximum -- the arithmetic of k_decode_combine (fast_kernels.py:238-253),
// eight splits' loads in flight at a time. merge_partials: lane (r16, g) gets dims 16dt + 4g + i of head
// r16; merge_partial_elem: one (head, dim) element, out = num / den.
__device__ __forceinline__ void merge_partials(rsrc_t acc_r, rsrc_t ml_r, int head, int g, int ns, float sl2,
                                               f32x4 (&num)[4], float &den) {
  constexpr int SB = 8;
  float M = kNegInf;
  den = 0.f;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) num[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < ns; s0 += SB) {
    float mv[SB], lv[SB];
    f32x4 av[SB][4];
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      const uint32_t e = (uint32_t)(head * ns + min(s0 + i, ns - 1));
      mv[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ml_r, e * 8, 0, kSC1));
      lv[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ml_r, e * 8 + 4u, 0, kSC1));
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        av[i][dt] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(acc_r, (e * 64 + 16 * dt + 4 * g) * 4, 0, kSC1));
    }
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      if (s0 + i >= ns) break;
      if (mv[i] == kNegInf) continue;  // an empty split adds nothing
      if (mv[i] > M) {
        const float sc = (M == kNegInf) ? 0.f : fast_exp2((M - mv[i]) * sl2);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) num[dt] *= sc;
        den *= sc;
        M = mv[i];
      }
      const float wt = fast_exp2((mv[i] - M) * sl2);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) num[dt] += wt * av[i][dt];
      den += wt * lv[i];
    }
  }
}
__device__ __forceinline__ float merge_partial_elem(rsrc_t acc_r, rsrc_t ml_r, int head, int d, int ns, float sl2) {
  constexpr int SB = 8;
  float M = kNegInf, num = 0.f, den = 0.f;
  for (int s0 = 0; s0 < ns; s0 += SB) {
    float mv[SB], lv[SB], av[SB];
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      const uint32_t e = (uint32_t)(head * ns + min(s0 + i, ns - 1));
      mv[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ml_r, e * 8, 0, kSC1));
      lv[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ml_r, e * 8 + 4u, 0, kSC1));
      av[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(acc_r, (e * 64 + d) * 4, 0, kSC1));
    }
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      if (s0 + i >= ns) break;
      if (mv[i] == kNegInf) continue;
      if (mv[i] > M) {
        const float sc = (M == kNegInf) ? 0.f : fast_exp2((M - mv[i]) * sl2);
        num *= sc;
        den *= sc;
        M = mv[i];
      }
      const float wt = fast_exp2((mv[i] - M) * sl2);
      num += wt * av[i];
      den += wt * lv[i];
    }
  }
  return num / den;
}

}  // namespace a8
