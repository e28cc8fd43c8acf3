// Packed variable-length causal prefill attention at head_dim 128 (a8_prefill_attn with hd = 128).
//
// Semantics: those of prefill.hip (serve/fast_kernels.py:296-358, the reference's kernel with HD = 128): a
// block of <= 64 packed query rows [q0, q0+n) of one request at positions [p0, p0+n) of cache row `slot`,
// each row attending keys [0, p0+n) with key <= its position, online softmax in fp32, bf16 weights in P.V,
// out = bf16(acc / l).
//
// MI355X design: the head_dim-64 kernel's (prefill.hip) at twice the width, with the same LDS budget:
//   * One workgroup = one half block (32 query rows) x one kv head x a share of <= 4 of its q heads; its waves
//     are the q heads, two workgroups per compute unit (80 KB of LDS each, two waves per SIMD). A wave runs
//     its two 16-row query groups through every tile (the O^T accumulators of two groups are 64 VGPRs at 128
//     dims); the two halves of a block are separate workgroups with their own key ranges.
//   * Tiles of 32 keys (8 KB of K and 8 KB of V, as the head_dim-64 tile) go from HBM / L2 into LDS by DMA, in
//     a ring of three buffers (tiles t+1 and t+2 in flight while t is computed), this wave's requests spread
//     over its query groups, one barrier per tile. K is row-major (256 B rows) with the 16-byte chunks of row
//     r permuted by chunk ^ ((r & 3) | ((r >> 3) & 3) << 2), so the 16 key rows a 16-lane group reads for one
//     score product hit 16 distinct chunk positions; V's chunks by chunk ^ 2 (r & 3), read transposed by
//     ds_read_b64_tr_b16 (the layout of attn_cols.hip).
//   * Per (16-row group, tile): S^T = K . Q^T as 2 x 4 v_mfma_f32_16x16x32_bf16 (key rows 8g + 4tt + i of the
//     C layout, so that layout is the P^T operand of the next product), scores in exp2 units relative to a lazy
//     running offset (Q^T pre-scaled by scale * log2 e in LDS, the product started from -offset; raised only
//     when a score passes it by kPf128Lazy, or on the first tile when a column's max is below kPf128Low),
//     8 exp2 per lane, O^T += V^T . P^T (8 products) and the weights' column sums (1 product against ones).
//     The two groups are software-pipelined: group 1's score products run beside group 0's softmax, group 0's
//     P.V beside group 1's column max.
#include "decode_tile.h"

namespace a8 {
namespace {

constexpr int kPf128HW = 4;          // q heads (waves) per workgroup
constexpr int kPf128Keys = 32;       // keys per tile
constexpr uint32_t kRow128 = 256;    // bytes per cached key row
constexpr int kTile128 = kPf128Keys * 128;  // bf16 elements of one K or V tile (8 KB)
constexpr float kPf128Lazy = 8.f;
constexpr float kPf128Low = -64.f;
constexpr int UPW2 = 2;              // 16-row query groups per wave

// DMA instruction i (0..15) of the tile at key t0: i < 8 K rows 4i..4i+3 (1 KB), else V rows 4(i-8)...
// kb: this lane's K source offset inside 4 rows before the instruction's chunk permutation (bits 6-7 of the
// byte offset flip with (i >> 1) & 3); vb: its V source offset.
__device__ __forceinline__ void pf128_dma(int i, uint32_t t0, rsrc_t kr, rsrc_t vr, uint16_t *kt, uint16_t *vt,
                                          uint32_t kb, uint32_t vb) {
  const int j = i & 7;
  const uint32_t off = t0 * kRow128 + (uint32_t)j * 1024u;
  if (i < 8)
    bld16_lds<0>(kr, reinterpret_cast<char *>(kt) + j * 1024, off + (kb ^ (64u * (uint32_t)((j >> 1) & 3))), 0u);
  else
    bld16_lds<0>(vr, reinterpret_cast<char *>(vt) + j * 1024, off + vb, 0u);
}

template <int NW>
__global__ __launch_bounds__(64 * kPf128HW, 2) void k_prefill128(
    const uint16_t *__restrict__ q, int64_t s_qr, int64_t s_qh, int R,
    const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc, int64_t s_kb, int64_t s_kh,
    int cache_rows, int cache_len, uint16_t *__restrict__ out, int64_t s_or, int64_t s_oh,
    const int32_t *__restrict__ bq0, const int32_t *__restrict__ bn, const int32_t *__restrict__ bslot,
    const int32_t *__restrict__ bpos0, int group, int hsplit, int hpw, float sl2, int nh, int nblk_) {
  warm_kernargs<152>();  // the explicit arguments above span 0x00-0x97
  __shared__ __attribute__((aligned(16))) uint16_t kA[kTile128];
  __shared__ __attribute__((aligned(16))) uint16_t kB[kTile128];
  __shared__ __attribute__((aligned(16))) uint16_t kC[kTile128];
  __shared__ __attribute__((aligned(16))) uint16_t vA[kTile128];
  __shared__ __attribute__((aligned(16))) uint16_t vB[kTile128];
  __shared__ __attribute__((aligned(16))) uint16_t vC[kTile128];
  // Q^T operands: [wave][group][dim slice][lane] x 16 bytes (8 KB per wave)
  __shared__ __attribute__((aligned(16))) uint16_t qs[kPf128HW * UPW2 * 4 * 64 * 8];
  // Unit u = (block, kv head) in order; its 2 x hsplit workgroups (half block, head share) 8 apart, so all of
  // them run on one XCD and share the unit's tiles in its L2 (C4's shape: 83.0 -> 82.5 us against the halves
  // as separate units on neighbouring XCDs); the grid padded to whole runs of 8 units.
  const int nkv_ = nh / hsplit;
  const int nsh = 2 * hsplit;  // workgroups per (block, kv head): halves x head shares
  const int chunk = blockIdx.x / (8 * nsh), rem = blockIdx.x - chunk * (8 * nsh);
  const int sh = rem >> 3, u = chunk * 8 + (rem & 7);
  const int half = sh >= hsplit ? 1 : 0, hs = sh - half * hsplit;
  const int blk = u / nkv_, kh = u - blk * nkv_;
  if (blk >= nblk_) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int nw = NW;
  const int r16 = lane & 15, g = lane >> 4;

  // Block metadata is uniform over the workgroup: early exits before any barrier.
  const int n = bn[blk];
  if (n <= 0) return;
  const int q0 = bq0[blk], p0 = bpos0[blk];
  const int64_t sl = bslot[blk];
  if (sl < 0 || sl >= cache_rows || p0 < 0 || q0 < 0 || q0 >= R) return;
  const int nv = min(min(n, 64), R - q0) - 32 * half;  // valid query rows of this half
  if (nv <= 0) return;
  const int nvh = min(nv, 32);
  const int r0 = q0 + 32 * half, ph = p0 + 32 * half;  // the half's first row and its position
  const int hi = min(ph + nvh, cache_len);              // keys [0, hi)
  if (hi <= 0) return;
  const int ntile = (hi + kPf128Keys - 1) / kPf128Keys;

  const int64_t cb = sl * s_kb + (int64_t)kh * s_kh;
  const rsrc_t kr = make_rsrc(kc + cb, (uint32_t)hi * kRow128);
  const rsrc_t vr = make_rsrc(vc + cb, (uint32_t)hi * kRow128);
  // DMA source offsets of this lane (row lane / 16 of each 4-row instruction, LDS chunk lane % 16)
  const uint32_t dr = (uint32_t)(lane >> 4), dc = (uint32_t)(lane & 15);
  const uint32_t kb = dr * kRow128 + 16u * (dc ^ dr);
  const uint32_t vb = dr * kRow128 + 16u * (dc ^ (2u * dr));
  // K A-operand reads: tile row 8(r16/4) + 4tt + r16%4 (its chunk permutation is r16), chunk 4s + g
  const uint32_t krd = (uint32_t)(8 * (r16 >> 2) + (r16 & 3)) * kRow128;
  // V^T reads (attn_cols.hip's layout): row 8g + r16/4 (+4), chunk (2dt + (r16%4)/2) ^ 2 ((r16/4) & 3),
  // half r16 % 2
  const uint32_t vrr = (uint32_t)(r16 >> 2), vperm = 2u * (vrr & 3u), vhalf = (uint32_t)(r16 & 1) * 8u;
  const uint32_t vc0 = (uint32_t)((r16 & 3) >> 1);
  const uint32_t vrow = (8u * (uint32_t)g + vrr) * kRow128 + vhalf;

  const int gi = hs * hpw + w;  // this wave's q head within the kv head's group
  const bool active = gi < group;
  const int head = kh * group + gi;
  uint16_t *qw = qs + w * (UPW2 * 4 * 64 * 8) + lane * 8;
  f32x4 o[UPW2][8];  // O^T rows d = 16dt + 4g + i, column = query row 16k + r16 of the half
  float mcs[UPW2];
  f32x4 cneg[UPW2], lacc[UPW2];
  u32x4 ones;
  asm volatile("v_mov_b32 %0, 0x3f803f80" : "=v"(ones[0]));
  ones[1] = ones[0];
  ones[2] = ones[0];
  ones[3] = ones[0];
  // Q^T by DMA (requested before the first K / V tiles): request (k, s) reads dims 32s + 8g.. of the half's
  // row 16k + r16; rows past nvh read as zeros (the buffer ends at row nvh - 1; the host keeps s_qr >= 128).
  if (active) {
    const rsrc_t qrs = make_rsrc(q + (int64_t)r0 * s_qr + (int64_t)head * s_qh,
                                 (uint32_t)((int64_t)(nvh - 1) * s_qr * 2 + 256));
#pragma unroll
    for (int k = 0; k < UPW2; ++k)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        bld16_lds<0>(qrs, reinterpret_cast<char *>(qs) + (w * 8 + 4 * k + s) * 1024,
                     (uint32_t)(((int64_t)(16 * k + r16) * s_qr + 32 * s + 8 * g) * 2), 0u);
  }
#pragma unroll
  for (int k = 0; k < UPW2; ++k) {
    mcs[k] = 0.f;
    cneg[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    lacc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[k][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  auto issue = [&](int t, uint16_t *kt, uint16_t *vt) __attribute__((always_inline)) {
    for (int i = w; i < 16; i += nw) pf128_dma(i, (uint32_t)(kPf128Keys * t), kr, vr, kt, vt, kb, vb);
  };
  // this wave's share of tile t complete (the next tile's share may stay in flight: at least 16 / nw
  // requests a tile per wave), then meet
  auto ready = [&](bool ahead) __attribute__((always_inline)) {
    if (ahead) {
      if (nw == 1) __builtin_amdgcn_s_waitcnt(0x4F70);  // s_waitcnt vmcnt(16 / nw)
      if (nw == 2) __builtin_amdgcn_s_waitcnt(0x0F78);
      if (nw == 3) __builtin_amdgcn_s_waitcnt(0x0F75);
      if (nw == 4) __builtin_amdgcn_s_waitcnt(0x0F74);
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    lds_barrier();
  };
  // S^T of query group k (8 products in two chains of 4)
  auto scores = [&](int k, const u32x4 (&ka)[2][4], f32x4 (&s)[2]) __attribute__((always_inline)) {
    u32x4 qb[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) qb[d] = ld16(qw + (4 * k + d) * 64 * 8);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x4 a = mfma16x16x32(ka[tt][0], qb[0], cneg[k]);
#pragma unroll
      for (int d = 1; d < 4; ++d) a = mfma16x16x32(ka[tt][d], qb[d], a);
      s[tt] = a;
    }
  };
  // O^T += V^T . P^T for group k, and the column sums (9 products)
  auto weigh = [&](int k, const u32x4 (&va)[8], u32x4 pB) __attribute__((always_inline)) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[k][dt] = mfma16x16x32(va[dt], pB, o[k][dt]);
    lacc[k] = mfma16x16x32(ones, pB, lacc[k]);
  };
  auto compute = [&](auto masked_tag, int t, const uint16_t *kt, const uint16_t *vtile, auto issue_tag, int tn,
                     uint16_t *kn, uint16_t *vn) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool ISSUE = decltype(issue_tag)::value;
    if (!active) {
      if (ISSUE) issue(tn, kn, vn);
      return;
    }
    const int kt0 = kPf128Keys * t;
    u32x4 ka[2][4], va[8];
    const char *kp = reinterpret_cast<const char *>(kt);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int d = 0; d < 4; ++d) ka[tt][d] = ld16(kp + krd + 4u * tt * kRow128 + 16u * ((4u * d + g) ^ r16));
    const char *vp = reinterpret_cast<const char *>(vtile) + vrow;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const char *p = vp + (((2u * dt + vc0) ^ vperm) << 4);
      const u32x2 lo = lds_tr16(p), hi2 = lds_tr16(p + 4 * kRow128);
      va[dt] = u32x4{lo[0], lo[1], hi2[0], hi2[1]};
    }
    f32x4 s[2];
    u32x4 pP;  // the previous group's weights
    scores(0, ka, s);
#pragma unroll
    for (int k = 0; k < UPW2; ++k) {
      if (ISSUE)  // this wave's instructions w + nw j with j = k mod 2
#pragma unroll
        for (int j = k; j * nw < 16; j += 2)
          if (16 % nw == 0 || w + nw * j < 16) pf128_dma(w + nw * j, (uint32_t)(kPf128Keys * tn), kr, vr, kn, vn, kb, vb);
      if (MASKED) {
        // keys <= the query position (and < hi): key kt0 + 8g + 4tt + i of this lane against one threshold
        const int d = min(ph + 16 * k + r16, hi - 1) - kt0 - 8 * g;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (4 * tt + i > d) s[tt][i] = kNegInf;
      }
      // group k's max over its 8 scores, beside group k-1's products
      float m1 = 0.f, m2 = 0.f, mt = 0.f;
#pragma unroll
      for (int j = 0; j < 9; ++j) {
        if (k > 0) {
          if (j < 8) o[k - 1][j] = mfma16x16x32(va[j], pP, o[k - 1][j]);
          else lacc[k - 1] = mfma16x16x32(ones, pP, lacc[k - 1]);
        }
        if (j == 0) m1 = max3_ieee(s[0][0], s[0][1], s[0][2]);
        else if (j == 1) m2 = max3_ieee(s[0][3], s[1][0], s[1][1]);
        else if (j == 2) mt = max3_ieee(m1, m2, max_ieee(s[1][2], s[1][3]));
        __builtin_amdgcn_sched_barrier(0);
      }
      // the lazy offset (as prefill.hip): raised when a lane group's max passes it by more than kPf128Lazy, or
      // on the block's first tile (key 0 is visible to every row) when it is below kPf128Low
      const bool first = kt0 == 0;
      if (__ballot(mt > kPf128Lazy || mt < (first ? kPf128Low : kNegInf))) {
        const float tm = max_over_groups_ieee(mt);
        const float up = first ? tm : fmaxf(tm, 0.f);
        const float alpha = first ? 0.f : fast_exp2(-up);
        lacc[k] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[k][dt] *= alpha;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) s[tt] -= up;
        mcs[k] += up;
        cneg[k] = f32x4{-mcs[k], -mcs[k], -mcs[k], -mcs[k]};
      }
      // group k's weights, beside group k+1's score products
      u32x4 qn[4];
      if (k + 1 < UPW2)
#pragma unroll
        for (int d = 0; d < 4; ++d) qn[d] = ld16(qw + (4 * (k + 1) + d) * 64 * 8);
      f32x4 sn[2];
      u32x4 pB;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        if (k + 1 < UPW2) sn[tt] = mfma16x16x32(ka[tt][0], qn[0], cneg[k + 1]);
        const float e0 = fast_exp2(s[tt][0]), e1 = fast_exp2(s[tt][1]);
        pB[2 * tt] = pack_bf16x2(e0, e1);
        __builtin_amdgcn_sched_barrier(0);
        if (k + 1 < UPW2) sn[tt] = mfma16x16x32(ka[tt][1], qn[1], sn[tt]);
        const float e2 = fast_exp2(s[tt][2]), e3 = fast_exp2(s[tt][3]);
        pB[2 * tt + 1] = pack_bf16x2(e2, e3);
        __builtin_amdgcn_sched_barrier(0);
        if (k + 1 < UPW2) {
          sn[tt] = mfma16x16x32(ka[tt][2], qn[2], sn[tt]);
          sn[tt] = mfma16x16x32(ka[tt][3], qn[3], sn[tt]);
        }
      }
      pP = pB;
      if (k + 1 < UPW2) {
        s[0] = sn[0];
        s[1] = sn[1];
      }
    }
    weigh(UPW2 - 1, va, pP);
  };

  // tiles [0, nfull) lie wholly at or below the half's first position (every row sees every key) and inside
  // the range; the rest -- at most two of 32 keys -- cross the diagonal. Tile t sits in buffer t % 3.
  const int nfull = min(max((ph + 1) / kPf128Keys, 0), hi / kPf128Keys);
  issue(0, kA, vA);
  if (ntile > 1) issue(1, kB, vB);
  // the Q^T operands times sl2, rounded to bf16, in place, once their DMA has landed (before this wave's
  // share of tile 0: at least 16 / NW requests after it)
  if (active) {
    wait_vmcnt<16 / NW>();
#pragma unroll
    for (int j = 0; j < 4 * UPW2; ++j) {
      uint16_t *p = qw + j * 64 * 8;
      u32x4 v = ld16(p);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = pack_bf16x2(bf_lo(v[e]) * sl2, bf_hi(v[e]) * sl2);
      st16(p, v);
    }
  }
  // wave priority as in prefill.hip: 1 while more than half of the tiles remain
  auto prio = [&](int left) __attribute__((always_inline)) {
    if (2 * left > ntile) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
  };
  int t = 0;
  if (nfull > 0) {
    for (;; t += 3) {
      prio(ntile - t);
      ready(t + 1 < ntile);
      compute(std::false_type{}, t, kA, vA, std::true_type{}, t + 2, kC, vC);
      if (t + 1 >= nfull) {
        t += 1;
        break;
      }
      prio(ntile - t - 1);
      ready(t + 2 < ntile);
      compute(std::false_type{}, t + 1, kB, vB, std::true_type{}, t + 3, kA, vA);
      if (t + 2 >= nfull) {
        t += 2;
        break;
      }
      prio(ntile - t - 2);
      ready(t + 3 < ntile);
      compute(std::false_type{}, t + 2, kC, vC, std::true_type{}, t + 4, kB, vB);
      if (t + 3 >= nfull) {
        t += 3;
        break;
      }
    }
  }
  for (; t < ntile; ++t) {
    prio(ntile - t);
    ready(false);
    const int bsel = t % 3;
    const uint16_t *kt = bsel == 0 ? kA : bsel == 1 ? kB : kC;
    const uint16_t *vtb = bsel == 0 ? vA : bsel == 1 ? vB : vC;
    compute(std::true_type{}, t, kt, vtb, std::false_type{}, 0, kA, vA);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // the last request (zeros past the range) lands before the end

  if (!active) return;
#pragma unroll
  for (int k = 0; k < UPW2; ++k) {
    const int mrow = 16 * k + r16;
    if (mrow >= nvh) continue;
    const float rl = __builtin_amdgcn_rcpf(lacc[k][0]);  // l >= 2^kPf128Low for a live row
    uint16_t *op = out + (int64_t)(r0 + mrow) * s_or + (int64_t)head * s_oh + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      st8(op + 16 * dt, u32x2{pack_bf16x2(o[k][dt][0] * rl, o[k][dt][1] * rl),
                              pack_bf16x2(o[k][dt][2] * rl, o[k][dt][3] * rl)});
  }
}

}  // namespace

// The head_dim-128 launch behind a8_prefill_attn (arguments checked there: pointers, alignment, s_ks = hd,
// bm = 64, nq % group == 0).
int prefill128(const void *q, int64_t s_qr, int64_t s_qh, int R, const void *kc, const void *vc, int64_t s_kb,
               int64_t s_kh, int cache_rows, int cache_len, void *out, int64_t s_or, int64_t s_oh, const int32_t *bq0,
               const int32_t *bn, const int32_t *bslot, const int32_t *bpos0, int nblk, int nq, int group,
               float scale, hipStream_t stream) {
  const int nkv = nq / group;
  const int hpw = group < kPf128HW ? group : kPf128HW;
  const int hsplit = (group + hpw - 1) / hpw;
  const int nh = nkv * hsplit;
  if (s_qr < 128 || s_qr >= (1 << 24))  // the Q requests' 32-bit byte offsets (31 rows) and their row range
    return set_error(A8_EUNSUP, "prefill_attn: q row stride %lld outside [128, 2^24)", (long long)s_qr);
  if ((int64_t)cache_len * kRow128 >= ((int64_t)1 << 32))
    return set_error(A8_EUNSUP, "prefill_attn: cache of %d positions too long for 32-bit offsets", cache_len);
  const int64_t grid = ((int64_t)nblk * nkv + 7) / 8 * 8 * 2 * hsplit;
  if (grid * 64 * hpw > (int64_t)UINT32_MAX)
    return set_error(A8_EUNSUP, "prefill_attn: too many blocks x heads (%d x %d)", nblk, nh);
  static_assert(kPf128HW == 4, "one instantiation per workgroup size");
  auto kern = hpw == 1 ? k_prefill128<1> : hpw == 2 ? k_prefill128<2> : hpw == 3 ? k_prefill128<3> : k_prefill128<4>;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * hpw), 0, stream, (const uint16_t *)q, s_qr, s_qh, R,
                     (const uint16_t *)kc, (const uint16_t *)vc, s_kb, s_kh, cache_rows, cache_len, (uint16_t *)out,
                     s_or, s_oh, bq0, bn, bslot, bpos0, group, hsplit, hpw, scale * kLog2e, nh, nblk);
  return (int)hipGetLastError();
}

}  // namespace a8
