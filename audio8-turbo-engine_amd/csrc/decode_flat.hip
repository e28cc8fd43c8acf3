// Balanced single-launch decode (a8_decode_attn_flat, a8_store_decode_flat, a8_decode_choose_flat): the
// decode attention of serve/fast_kernels.py:193-290 -- and, fused, the bias_rope_store before it
// (139-187) -- in one launch for any mix of row lengths.
//
// The split + combine pair needs three launches per layer with the store (store, split, combine), each
// a launch gap and at least one memory round trip, and a split count fixed per call leaves ragged rows
// unbalanced. Here:
//   * The work is partitioned by the actual lengths, on the device. Every workgroup reads the rows'
//     lengths and cache rows into LDS and scans them: row r has T_r = max(1, ceil(L_r / 64)) tiles per
//     kv head (an empty or unmapped row still counts one tile, whose 0/0 output is NaN as in the
//     reference), and unit (r, kh) owns the flat tiles [nkv P_r + kh T_r, + T_r), P_r = sum of T
//     before r. W = min(grid * 4, N) waves split the N flat tiles evenly: wave k takes [N k / W,
//     N (k+1) / W), at least one tile.
//   * A wave walks its range unit by unit (one segment per unit), with the decode's two-stage tile
//     pipeline (decode_tile.h) running across segment boundaries and each segment's q -- or qkv rows,
//     fused -- requested one segment ahead. A segment that is a whole unit writes `out` directly.
//   * A unit spread over several waves: each writes its (acc, m, l) partial to a fixed workspace slot
//     (2k for wave k's first segment, 2k + 1 for its last) with device-coherent stores, waits for them
//     to complete and counts itself in with an atomic on the unit's counter. The wave that arrives last
//     merges the unit's partials (device-coherent loads) in wave order -- so the bits do not depend on
//     which wave merges -- writes `out` and puts the counter back to zero for the next launch. No wave
//     waits for another.
//   * Fused: the wave holding a unit's first tile also does the unit's store (k / v, and q when asked
//     for); every segment computes its q from qkv + bias + RoPE (fused_qkv.h), and the tile holding the
//     new key takes it from registers.
#include "decode_tile.h"
#include "fused_qkv.h"

namespace a8 {

constexpr int kFlatNW = 4;          // waves per workgroup
constexpr int kFlatMaxRows = 2048;  // rows per call: the per-row metadata lives in LDS
constexpr int kFlatMaxGrid = 1024;  // with fewer than 2^20 tiles, the partition arithmetic fits 32 bits
constexpr int kFlatMaxTiles = 1 << 20;

// Inclusive prefix sum over the 64 lanes with DPP moves (no LDS round trip): Hillis-Steele within each
// 16-lane row (row_shr 1, 2, 4, 8; lanes shifted in from outside the row add 0), then row_bcast:15 adds
// lane 15 of rows 0 / 2 to rows 1 / 3 and row_bcast:31 adds lane 31 to rows 2 and 3.
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);
  return v;
}

template <bool FUSED>
__global__ __launch_bounds__(64 * kFlatNW, 1) void k_decode_flat(
    const uint16_t *__restrict__ q, int64_t s_qb, int64_t s_qh, uint16_t *kc, uint16_t *vc, int64_t s_kb,
    int64_t s_kh, int64_t s_ks, int cache_rows, int cache_len, const int32_t *__restrict__ lens,
    const int32_t *__restrict__ rowmap, uint16_t *__restrict__ out, int64_t s_ob, int64_t s_oh,
    float *__restrict__ acc_ws, float *__restrict__ ml_ws, int32_t *__restrict__ counters, int b, int nq,
    int nkv, int group, float sl2, StoreIn si) {
  warm_kernargs<264>();  // the explicit arguments above span 0x000-0x107
  __shared__ int m_pre[kFlatMaxRows + 1];  // tiles per kv head before row r
  __shared__ int m_len[kFlatMaxRows];      // keys attended by row r (0: empty or unmapped)
  __shared__ int m_crow[kFlatMaxRows];     // cache row attended by row r (-1: outside the cache)
  __shared__ int m_pos[FUSED ? kFlatMaxRows : 1];
  __shared__ int m_slot[FUSED ? kFlatMaxRows : 1];
  __shared__ __attribute__((aligned(16))) uint16_t vbA[kFlatNW * kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t vbB[kFlatNW * kVTile];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  for (int r = tid; r < b; r += 64 * kFlatNW) {
    const int crow = rowmap ? rowmap[r] : r;
    const bool ok = crow >= 0 && crow < cache_rows;
    const int L = ok ? min(max(lens[r], 0), cache_len) : 0;
    m_len[r] = L;
    m_crow[r] = ok ? crow : -1;
    m_pre[r + 1] = max(1, (L + 63) >> 6);
    if (FUSED) {
      m_pos[r] = si.pos[r];
      m_slot[r] = si.slot[r];
    }
  }
  __syncthreads();
  if (w == 0) {  // prefix sums of the tile counts: lane l sums its block of c rows, one wave scan
    const int c = (b + 63) >> 6;
    const int lo = lane * c, hi = min(lo + c, b);
    int tot = 0;
    for (int r = lo; r < hi; ++r) tot += m_pre[r + 1];
    int run = wave_incl_scan(tot) - tot;
    for (int r = lo; r < hi; ++r) {
      run += m_pre[r + 1];
      m_pre[r + 1] = run;
    }
    if (lane == 0) m_pre[0] = 0;
  }
  __syncthreads();

  // W waves take part, never more than there are tiles: then every one of them holds at least one tile,
  // and the waves over a unit's tiles are exactly kf..kl (its contributors). The others leave.
  // N < 2^20 tiles and W <= 4096 waves (checked at the entry): every product below fits 32 bits.
  const uint32_t N = (uint32_t)(nkv * m_pre[b]);
  const uint32_t W = min((uint32_t)gridDim.x * kFlatNW, N);
  const uint32_t k = (uint32_t)blockIdx.x * kFlatNW + (uint32_t)w;
  if (k >= W) return;  // no barrier follows
  const uint32_t nq_w = N / W, nr_w = N % W;  // N k / W = k nq_w + k nr_w / W, with k nr_w < 2^24
  const int t0 = (int)(k * nq_w + (k * nr_w) / W), t1 = (int)((k + 1) * nq_w + ((k + 1) * nr_w) / W);
  // the wave holding flat tile t
  auto wave_of = [&](int t) { return (int)(((uint32_t)(t + 1) * W - 1) / N); };

  // first row: the rows whose tiles all end at or before t0
  int r0 = 0;
  for (int base = 0; base < b; base += 64) {
    const int r = base + lane;
    r0 += __popcll(__ballot(r < b && nkv * m_pre[r + 1] <= t0));
  }
  r0 = __builtin_amdgcn_readfirstlane(r0);

  struct Unit {
    int r, kh, us, T, L, crow, p, srow;
    rsrc_t kr, vr;
  };
  auto unit_at = [&](int r, int kh, Unit &u) {
    r = min(r, b - 1);  // always true of a consistent partition; keeps every address in bounds regardless
    const int pre = __builtin_amdgcn_readfirstlane(m_pre[r]);
    const int T = __builtin_amdgcn_readfirstlane(m_pre[r + 1]) - pre;
    u.r = r;
    u.kh = kh;
    u.T = T;
    u.us = nkv * pre + kh * T;
    u.L = __builtin_amdgcn_readfirstlane(m_len[r]);
    u.crow = __builtin_amdgcn_readfirstlane(m_crow[r]);
    u.p = FUSED ? __builtin_amdgcn_readfirstlane(m_pos[r]) : 0;
    u.srow = FUSED ? __builtin_amdgcn_readfirstlane(m_slot[r]) : 0;
    const int64_t cb = (int64_t)(u.crow >= 0 ? u.crow : 0) * s_kb + (int64_t)kh * s_kh;
    u.kr = make_rsrc(kc + cb, (uint32_t)u.L * kRow);  // keys past L read zeros, nothing is fetched
    u.vr = make_rsrc(vc + cb, (uint32_t)u.L * kRow);
  };
  auto next_unit = [&](const Unit &u, Unit &n) {
    if (u.kh + 1 < nkv)
      unit_at(u.r, u.kh + 1, n);
    else
      unit_at(u.r + 1, 0, n);
  };

  TileLane tl;
  tl.init(lane);
  uint16_t *va = vbA + w * kVTile, *vb = vbB + w * kVTile;
  // the 2W partial slots: group x 64 floats of acc and group x 2 of (m, l) each
  const rsrc_t acc_r = make_rsrc(acc_ws, 2u * W * (uint32_t)group * 64u * 4u);
  const rsrc_t ml_r = make_rsrc(ml_ws, 2u * W * (uint32_t)group * 2u * 4u);
  const rsrc_t none = make_rsrc(kc, 0u);

  // raw q of a unit, requested one segment ahead: the q rows (decode) or the qkv / bias / table chunks
  // (fused)
  u32x4 rq0, rq1;
  QkvRaw rx;
  auto request_q = [&](const Unit &u) {
    if (FUSED) {
      load_qkv_raw(si, true, u.r, u.kh, u.p, group, nq, nkv, tl, rx);
    } else {
      const rsrc_t qr = make_rsrc_wave(q + (int64_t)u.r * s_qb + (int64_t)u.kh * group * s_qh,
                                       (uint32_t)(group * s_qh * 2));
      const uint32_t qo = (uint32_t)(tl.r16 * s_qh * 2) + 16u * tl.g;
      rq0 = bld16(qr, qo);
      rq1 = bld16(qr, qo + 64u);
    }
  };

  Unit cu, nu;
  {
    const int pre = __builtin_amdgcn_readfirstlane(m_pre[r0]);
    const int T = __builtin_amdgcn_readfirstlane(m_pre[r0 + 1]) - pre;
    unit_at(r0, min((t0 - nkv * pre) / T, nkv - 1), cu);
  }
  nu = cu;
  KTile A[1], B[1];
  load_step<1>(A, va, cu.kr, cu.vr, (uint32_t)(64 * (t0 - cu.us)), tl);
  request_q(cu);

  SoftmaxState S;
  S.reset();
  u32x4 qc0, qc1;
  KVPatch pt;
  pt.col = -1;
  int t = t0, seg_lo = t0;
  bool fresh = true, first_seg = true;

  // End of a segment [seg_lo, seg_hi) of unit u: the output, or a partial and the merge by the last
  // wave to arrive.
  auto finish = [&](const Unit &u, int seg_hi) {
    const float lsum = sum_over_groups(S.lsum);
    const bool mine = tl.r16 < group;
    const int hq = u.kh * group + tl.r16;
    if (seg_lo == u.us && seg_hi == u.us + u.T) {
      if (mine) {
        uint16_t *o = out + (int64_t)u.r * s_ob + (int64_t)hq * s_oh + 4 * tl.g;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
          st8(o + 16 * dt, u32x2{pack_bf16x2(S.o[dt][0] / lsum, S.o[dt][1] / lsum),
                                 pack_bf16x2(S.o[dt][2] / lsum, S.o[dt][3] / lsum)});
      }
      return;
    }
    // The partial goes out with agent-coherent (sc1) stores, which write through the XCD's L2; once they
    // have completed (vmcnt(0)) the counter atomic makes the wave's arrival known. The merging wave reads
    // partials with sc1 loads issued after its atomic returned. Only the bytes exchanged here are kept
    // coherent: an agent-scope fence would write back and invalidate the whole L2 instead, for every
    // partial, while the other waves stream through it.
    const int64_t slot = 2 * (int64_t)k + (first_seg ? 0 : 1);
    if (mine) {
      const uint32_t ao = (uint32_t)(((slot * group + tl.r16) * 64 + 4 * tl.g) * 4);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, S.o[dt]), acc_r, ao + 64u * dt, 0, kSC1);
      if (tl.g == 0) {
        const uint32_t mo = (uint32_t)((slot * group + tl.r16) * 2 * 4);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(S.m), ml_r, mo, 0, kSC1);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(lsum), ml_r, mo + 4u, 0, kSC1);
      }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the partial has reached the coherent level
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const int uidx = u.r * nkv + u.kh;
    int old = 0;
    if (lane == 0) old = atomicAdd(counters + uidx, 1);
    old = __shfl(old, 0);
    const int kf = wave_of(u.us), kl = wave_of(u.us + u.T - 1);
    if (old != kl - kf) return;
    if (mine) {
      // the unit's partials in wave order, four waves' loads in flight at a time; every sum runs in wave
      // order. Wave kk's segment is its first one (slot 2kk) when its range starts inside the unit, which
      // holds for every wave after kf; wave kf's is its last (2kf + 1) when its range starts before.
      const int kf_last = (N * (uint32_t)kf < (uint32_t)u.us * W) ? 1 : 0;
      auto slot_of = [&](int kk) { return 2 * (int64_t)kk + (kk == kf ? kf_last : 0); };
      auto m_at = [&](int64_t sl, int e) {
        return __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(ml_r, (uint32_t)(((sl * group + tl.r16) * 2 + e) * 4), 0, kSC1));
      };
      // one pass with a running maximum (the weights of earlier partials are rescaled when it grows),
      // eight waves' loads in flight at a time: a unit over at most eight waves costs one round trip
      constexpr int MB = 8;
      float M = kNegInf, den = 0.f;
      f32x4 num[4] = {};
      for (int kb = kf; kb <= kl; kb += MB) {
        float mv[MB], lv[MB];
        f32x4 av[MB][4];
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          const int64_t sl = slot_of(min(kb + i, kl));
          mv[i] = m_at(sl, 0);
          lv[i] = m_at(sl, 1);
          const uint32_t ao = (uint32_t)(((sl * group + tl.r16) * 64 + 4 * tl.g) * 4);
#pragma unroll
          for (int dt = 0; dt < 4; ++dt)
            av[i][dt] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(acc_r, ao + 64u * dt, 0, kSC1));
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          if (kb + i > kl) break;
          if (mv[i] == kNegInf) continue;  // a partial with no finite score adds nothing
          if (mv[i] > M) {
            const float sc = (M == kNegInf) ? 0.f : fast_exp2((M - mv[i]) * sl2);
            den *= sc;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) num[dt] *= sc;
            M = mv[i];
          }
          const float wt = fast_exp2((mv[i] - M) * sl2);
          den += wt * lv[i];
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) num[dt] += wt * av[i][dt];
        }
      }
      uint16_t *o = out + (int64_t)u.r * s_ob + (int64_t)hq * s_oh + 4 * tl.g;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        st8(o + 16 * dt, u32x2{pack_bf16x2(num[dt][0] / den, num[dt][1] / den),
                               pack_bf16x2(num[dt][2] / den, num[dt][3] / den)});
    }
    if (lane == 0) counters[uidx] = 0;
  };

  // Consumes tile t from X after requesting tile t + 1 into Y.
  auto step = [&](KTile (&X)[1], uint16_t *xv, KTile (&Y)[1], uint16_t *yv) __attribute__((always_inline)) -> bool {
    const int tn = t + 1;
    const bool more = tn < t1;
    const bool cross = more && tn == cu.us + cu.T;  // tile tn opens the next unit
    if (cross) next_unit(cu, nu);
    {
      // one load sequence for every case (operands selected)
      const rsrc_t kr = !more ? none : cross ? nu.kr : cu.kr;
      const rsrc_t vr = !more ? none : cross ? nu.vr : cu.vr;
      const int off = (more && !cross) ? 64 * (tn - cu.us) : 0;
      load_step<1>(Y, yv, kr, vr, (uint32_t)off, tl);
    }
    if (fresh) {
      if (FUSED) {
        apply_qkv_raw(si, rx, true, cu.r, cu.kh, cu.p, cu.srow, cu.crow, cache_rows, cache_len, group, kc, vc, s_kb,
                      s_kh, s_ks, /*store=*/t == cu.us, tl, qc0, qc1, pt);
      } else {
        qc0 = rq0;
        qc1 = rq1;
      }
      if (cu.us + cu.T < t1) {  // the next segment's q, one segment ahead
        Unit n2;
        next_unit(cu, n2);
        request_q(n2);
      }
      fresh = false;
    }
    const int key0 = 64 * (t - cu.us);
    if (key0 < cu.L) compute_step<1, 16, FUSED>(X, xv, key0, cu.L, qc0, qc1, sl2, S, tl, lane, &pt);
    if (!more || cross) {
      finish(cu, tn);
      S.reset();
      first_seg = false;
      fresh = true;
      seg_lo = tn;
      if (cross) cu = nu;
    }
    t = tn;
    return more;
  };
  for (;;) {
    if (!step(A, va, B, vb)) break;
    if (!step(B, vb, A, va)) break;
  }
  // the request past the last tile still writes (zeros) into LDS: let it land before the wave ends.
  // s_waitcnt vmcnt(0).
  __builtin_amdgcn_s_waitcnt(0x0F70);
}

static inline bool al16f(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Body of a8_decode_attn_flat and a8_store_decode_flat (fused = si.qkv != nullptr).
static int flat_entry(const char *fn, const void *q, int64_t s_qb, int64_t s_qh, void *kc, void *vc, int64_t s_kb,
                      int64_t s_kh, int64_t s_ks, int cache_rows, int cache_len, const int32_t *lens,
                      const int32_t *rowmap, void *out, int64_t s_ob, int64_t s_oh, float *acc_ws, float *ml_ws,
                      int64_t ws_row_splits, int32_t *counters, int64_t n_counters, int b, int nq, int nkv, int hd,
                      int grid, float scale, const StoreIn &si, void *stream) {
  const bool fused = si.qkv != nullptr;
  if (hd != 64 && (fused || hd != 128))
    return set_error(A8_EUNSUP, "%s: head_dim %d not supported (64; 128 through the unfused call)", fn, hd);
  if (b < 0 || nq <= 0 || nkv <= 0 || nq % nkv || cache_rows < 0 || cache_len < 0)
    return set_error(A8_EINVAL, "%s: bad sizes b=%d nq=%d nkv=%d", fn, b, nq, nkv);
  const int group = nq / nkv;
  if (group > (fused ? kLaneK : 16))
    return set_error(A8_EUNSUP, "%s: GQA group %d > %d not supported", fn, group, fused ? kLaneK : 16);
  if (b > kFlatMaxRows) return set_error(A8_EUNSUP, "%s: %d rows > %d per call", fn, b, kFlatMaxRows);
  if (grid < 1 || grid > kFlatMaxGrid) return set_error(A8_EINVAL, "%s: grid %d out of range", fn, grid);
  if (b == 0) return 0;
  if ((!fused && !q) || !kc || !vc || !lens || !out || !acc_ws || !ml_ws || !counters)
    return set_error(A8_EINVAL, "%s: null pointer", fn);
  const int64_t tiles_max = (int64_t)nkv * b * (cache_len > 64 ? (cache_len + 63) / 64 : 1);
  if (tiles_max >= kFlatMaxTiles) return set_error(A8_EUNSUP, "%s: %lld key tiles > %d per call", fn,
                                                   (long long)tiles_max, kFlatMaxTiles);
  // partial slots: two per wave, group heads x 64 floats each, in a workspace of row-splits x nq x 64
  const int64_t W = (int64_t)grid * kFlatNW;
  if (2 * W > ws_row_splits * nkv)
    return set_error(A8_EWSPACE, "%s: workspace holds %lld row-splits, grid %d needs %lld", fn,
                     (long long)ws_row_splits, grid, (long long)((2 * W + nkv - 1) / nkv));
  if ((int64_t)b * nkv > n_counters)
    return set_error(A8_EWSPACE, "%s: %lld counters, need b*nkv = %lld", fn, (long long)n_counters,
                     (long long)b * nkv);
  if (s_ks != hd)
    return set_error(A8_EUNSUP, "%s: cache positions must be contiguous rows (s_ks %lld)", fn, (long long)s_ks);
  if ((!fused && !al16f(q)) || !al16f(kc) || !al16f(vc) || !al16f(out) || !al16f(acc_ws) ||
      ((fused ? 0 : (s_qb | s_qh)) | s_kb | s_kh | s_ks | s_ob | s_oh) & 7)
    return set_error(A8_EALIGN, "%s: pointers must be 16-byte aligned and strides multiples of 8", fn);
  if (hd != 64)  // the generic-head kernel (one launch, no workspace)
    return attn_cols_decode(fn, q, s_qb, s_qh, kc, vc, s_kb, s_kh, cache_rows, cache_len, lens, rowmap, out, s_ob,
                            s_oh, b, nq, nkv, hd, scale, (hipStream_t)stream);
  const hipStream_t st = (hipStream_t)stream;
  const float sl2 = scale * kLog2e;
  auto kern = fused ? k_decode_flat<true> : k_decode_flat<false>;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * kFlatNW), 0, st, (const uint16_t *)q, s_qb, s_qh, (uint16_t *)kc,
                     (uint16_t *)vc, s_kb, s_kh, s_ks, cache_rows, cache_len, lens, rowmap, (uint16_t *)out, s_ob,
                     s_oh, acc_ws, ml_ws, counters, b, nq, nkv, group, sl2, si);
  return (int)hipGetLastError();
}

}  // namespace a8

extern "C" int a8_decode_attn_flat(const void *q, int64_t s_qb, int64_t s_qh,
                                   const void *kc, const void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                                   int cache_rows, int cache_len, const int32_t *lens, const int32_t *rowmap,
                                   void *out, int64_t s_ob, int64_t s_oh,
                                   float *acc_ws, float *ml_ws, int64_t ws_row_splits,
                                   int32_t *counters, int64_t n_counters,
                                   int b, int nq, int nkv, int hd, int grid, float scale, void *stream) {
  using namespace a8;
  const StoreIn none{};
  return flat_entry("decode_attn_flat", q, s_qb, s_qh, const_cast<void *>(kc), const_cast<void *>(vc), s_kb, s_kh,
                    s_ks, cache_rows, cache_len, lens, rowmap, out, s_ob, s_oh, acc_ws, ml_ws, ws_row_splits,
                    counters, n_counters, b, nq, nkv, hd, grid, scale, none, stream);
}

extern "C" int a8_store_decode_flat(const void *qkv, int64_t s_qkv, const void *bias,
                                    const void *cos_tab, const void *sin_tab, int64_t s_cs, int n_tab,
                                    const int32_t *pos, const int32_t *slot,
                                    void *qo, int64_t s_qo_r, int64_t s_qo_h,
                                    void *kc, void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                                    int cache_rows, int cache_len, const int32_t *lens, const int32_t *rowmap,
                                    void *out, int64_t s_ob, int64_t s_oh,
                                    float *acc_ws, float *ml_ws, int64_t ws_row_splits,
                                    int32_t *counters, int64_t n_counters,
                                    int b, int nq, int nkv, int hd, int ring, int grid, float scale, void *stream) {
  using namespace a8;
  if (ring <= 0 || n_tab < 0) return set_error(A8_EINVAL, "store_decode_flat: bad ring %d / n_tab %d", ring, n_tab);
  if (b > 0 && (!qkv || !cos_tab || !sin_tab || !pos || !slot))
    return set_error(A8_EINVAL, "store_decode_flat: null pointer");
  if (b > 0 && (!al16f(qkv) || !al16f(cos_tab) || !al16f(sin_tab) || (bias && !al16f(bias)) || (qo && !al16f(qo)) ||
                (s_qkv | s_cs | (qo ? (s_qo_r | s_qo_h) : 0)) & 7))
    return set_error(A8_EALIGN, "store_decode_flat: pointers must be 16-byte aligned and strides multiples of 8");
  StoreIn si{};
  si.slot = slot;
  si.qkv = (const uint16_t *)qkv;
  si.s_qkv = s_qkv;
  si.bias = (const uint16_t *)bias;
  si.cos_tab = (const uint16_t *)cos_tab;
  si.sin_tab = (const uint16_t *)sin_tab;
  si.s_cs = s_cs;
  si.n_tab = n_tab;
  si.pos = pos;
  si.qo = (uint16_t *)qo;
  si.s_qo_r = s_qo_r;
  si.s_qo_h = s_qo_h;
  si.ring = ring;
  return flat_entry("store_decode_flat", nullptr, 0, 0, kc, vc, s_kb, s_kh, s_ks, cache_rows, cache_len, lens, rowmap,
                    out, s_ob, s_oh, acc_ws, ml_ws, ws_row_splits, counters, n_counters, b, nq, nkv, hd, grid,
                    scale, si, stream);
}

// Launch shape of the flat decode: enough waves for one tile each at the most keys the call can have
// (b rows x nkv x ceil(cache_len / 64) tiles), at most 4 per compute unit, and at most what the
// workspace's partial slots allow (two per wave).
extern "C" int a8_decode_choose_flat(int b, int nkv, int cache_len, int64_t cap_row_splits, int n_cu, int *grid_out) {
  using namespace a8;
  if (b < 1 || nkv < 1 || cache_len < 0 || n_cu < 1 || !grid_out)
    return set_error(A8_EINVAL, "decode_choose_flat: bad arguments b=%d nkv=%d n_cu=%d", b, nkv, n_cu);
  const int64_t tiles = (int64_t)b * nkv * (cache_len > 0 ? (cache_len + 63) / 64 : 1);
  int64_t grid = (tiles + kFlatNW - 1) / kFlatNW;
  if (grid > n_cu) grid = n_cu;
  if (grid > kFlatMaxGrid) grid = kFlatMaxGrid;
  const int64_t gmax = cap_row_splits * nkv / (2 * kFlatNW);
  if (grid > gmax) grid = gmax;
  if (grid < 1) return set_error(A8_EWSPACE, "decode_choose_flat: workspace of %lld row-splits is too small",
                                 (long long)cap_row_splits);
  *grid_out = (int)grid;
  return 0;
}
