// Split-K flash-decoding over the slot KV cache, GQA (a8_decode_attn, a8_decode_choose).
//
// Semantics follow serve/fast_kernels.py:193-290: query row b (one token, nq heads) attends keys
// [0, lens[b]) of cache row rowmap[b] (b when no rowmap); kv head kh serves q heads
// [kh*group, (kh+1)*group). The row's keys are cut into nsplit ranges of
// per = ceil(ceil(L/nsplit)/64)*64 keys (fast_kernels.py:207-209); each range produces a partial
// (acc, m, l) with an online softmax in fp32 and bf16 softmax weights in the P.V product, and the
// combine step merges the partials: w = exp(m - M) (0 for an empty range), out = sum(w acc)/sum(w l).
//
// MI355X design (the kernel streams ~512 B of K+V per key per row-layer from HBM; it is HBM bound):
//   * One workgroup = one (row, kv head, split); its `waves` wavefronts take the split's 64-key
//     tiles round-robin, each with its own online softmax, and merge through LDS at the end.
//   * K tiles are loaded straight into MFMA operand registers with 128-bit loads (one key row is
//     8 lanes x 16 B); S^T = K . Q^T runs on v_mfma_f32_16x16x32_bf16 with the group's q heads
//     (<= 16) as the 16 columns. The key rows of each 16x16 S^T tile are permuted so that the
//     C-layout of S^T is directly the B-operand layout of P^T (lane group g owns keys 8g..8g+7 of
//     each 32-key chunk) -- no shuffles between the two products.
//   * V tiles are loaded as 8 keys x 16 B per lane (each load instruction reads 8 whole 128-byte
//     key rows), transposed 8x8 in registers and written to a wave-private LDS tile V^T[d][key],
//     from where O^T += V^T . P^T reads 128-bit MFMA operands.
//   * Softmax statistics live per lane (column = q head); the max is reduced across the four
//     16-lane groups with cross-lane shuffles, the row sum is kept per lane group and reduced once.
//   * The tile machinery (loads, both products, online softmax) is in decode_tile.h. The running max
//     m is kept in raw score units (q.k) in the workspace, which only the decode kernels read; every
//     exponential is exp2((s - m) * scale * log2 e).
// This split + combine pair serves any nsplit the caller asks for; the default launch path is the
// streaming kernel of decode_stream.hip.
//
// FUSED (a8_store_decode_split): q and the new k / v come from qkv + bias + RoPE (fused_qkv.h, the
// store kernel's arithmetic) in every workgroup, split 0's first wave writes them to the cache (and q
// to qo) like k_bias_rope_store, and the tile holding the new key takes it from registers.
#include <mutex>

#include "decode_tile.h"
#include "fused_qkv.h"

namespace a8 {

template <int NW, bool FUSED>
__global__ __launch_bounds__(64 * NW, 2) void k_decode_split(
    const uint16_t *__restrict__ q, int64_t s_qb, int64_t s_qh,
    uint16_t *kc, uint16_t *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,  // written when FUSED
    int cache_rows, int cache_len, const int32_t *__restrict__ lens, const int32_t *__restrict__ rowmap,
    uint16_t *__restrict__ out, int64_t s_ob, int64_t s_oh, float *__restrict__ acc_ws,
    float *__restrict__ ml_ws, int32_t *__restrict__ counters, int nq, int nkv, int group, int ns, float scale_log2,
    StoreIn si) {
  warm_kernargs<256>();  // the explicit arguments above span 0x000-0x0ff and more
  // K and V tiles of the two pipeline buffers (one per wave each, load_tile_kv). Each read waits for its
  // tile's DMA with a counted vmcnt: the next tile's 16 requests are issued before the step.
  // (8 waves: K stays in registers, load_tile -- their K and V tiles would exceed the LDS)
  constexpr bool KL = NW <= 4;
  __shared__ __attribute__((aligned(16))) uint16_t kbA[KL ? NW * kVTile : 8];
  __shared__ __attribute__((aligned(16))) uint16_t kbB[KL ? NW * kVTile : 8];
  __shared__ __attribute__((aligned(16))) uint16_t vbA[NW * kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t vbB[NW * kVTile];
  const int sp = blockIdx.x, kh = blockIdx.y, row = blockIdx.z;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r16 = lane & 15, g = lane >> 4;

  int L = lens[row];
  const int crow = rowmap ? rowmap[row] : row;
  const int p = FUSED ? si.pos[row] : 0, srow = FUSED ? si.slot[row] : 0;
  if (crow < 0 || crow >= cache_rows) L = 0;  // no such cache row: attend nothing
  L = min(max(L, 0), cache_len);
  const int per = ((L + ns - 1) / ns + 63) / 64 * 64;
  const int lo = sp * per;
  const int hi = min(lo + per, L);

  constexpr uint32_t row_bytes = kRow;  // s_ks == 64, checked by the entry point
  TileLane tl;
  tl.init(lane);
  const int64_t cbase = (int64_t)(crow < 0 || crow >= cache_rows ? 0 : crow) * s_kb + (int64_t)kh * s_kh;
  // K / V of this (row, kv head) as buffers ending at key hi: rows past the range read as zeros.
  const rsrc_t kr = make_rsrc(kc + cbase, (uint32_t)hi * row_bytes);
  const rsrc_t vr = make_rsrc(vc + cbase, (uint32_t)hi * row_bytes);
  uint16_t *va = vbA + w * kVTile, *vb = vbB + w * kVTile;
  uint16_t *ka = kbA + (KL ? w * kVTile : 0), *kb = kbB + (KL ? w * kVTile : 0);
  KLdsLane kl;
  kl.init(lane);

  // Software pipeline over the wave's tiles first + k * 64*NW, k = 0..n-1, two register buffers, the
  // loads one tile ahead. The first tile is requested before the q / qkv prologue, so its latency and
  // the prologue's overlap (in the fused case the position being stored is patched from registers, so
  // the tile may be read before the store lands). The first step is peeled: the loop is entered with
  // exactly one tile's loads pending on both edges, so the compiler's waits stay partial (a load pending
  // only on the entry edge costs a full drain per iteration). Requests past the range read zeros
  // without memory traffic.
  constexpr int kStep = 64 * NW;
  const int first = lo + 64 * __builtin_amdgcn_readfirstlane(w);
  const int n = first < hi ? (hi - first + kStep - 1) / kStep : 0;
  KTile A[1], B[1];  // K operands: the tile in flight (registers) or read from LDS before its step
  auto load = [&](KTile &T, uint16_t *kt, uint16_t *vt, int t0) __attribute__((always_inline)) {
    if constexpr (KL)
      load_tile_kv(kt, vt, kr, vr, (uint32_t)t0, tl, kl);
    else
      load_tile(T, vt, kr, vr, (uint32_t)t0, tl);
  };
  auto kread = [&](KTile &T, const uint16_t *kt) __attribute__((always_inline)) {
    if constexpr (KL) read_k_tile<16>(T, kt, kl);  // the next tile's 16 requests went out after it
  };
  load(A[0], ka, va, first);

  // Q^T operand: column r16 = q head kh*group + r16 (zeros past the group).
  u32x4 qB0, qB1;
  KVPatch pt;
  pt.col = -1;
  if (FUSED) {
    QkvRaw rx;
    const int pu = __builtin_amdgcn_readfirstlane(p);
    load_qkv_raw(si, true, row, kh, pu, group, nq, nkv, tl, rx);
    apply_qkv_raw(si, rx, true, row, kh, pu, __builtin_amdgcn_readfirstlane(srow), __builtin_amdgcn_readfirstlane(crow),
                  cache_rows, cache_len, group, kc, vc, s_kb, s_kh, s_ks, /*store=*/sp == 0 && w == 0, tl, qB0, qB1, pt);
  } else {
    const rsrc_t qr = make_rsrc(q + (int64_t)row * s_qb + (int64_t)kh * group * s_qh, (uint32_t)(group * s_qh * 2));
    qB0 = bld16(qr, (uint32_t)(r16 * s_qh * 2) + 16u * g);
    qB1 = bld16(qr, (uint32_t)(r16 * s_qh * 2) + 16u * g + 64u);
  }
  SoftmaxState S;
  S.reset();

  if (n > 0) {
    load(B[0], kb, vb, first + kStep);
    kread(A[0], ka);
    compute_step<1, 16, FUSED>(A, va, first, hi, qB0, qB1, scale_log2, S, tl, lane, &pt);
    for (int k = 1; k < n; k += 2) {
      load(A[0], ka, va, first + (k + 1) * kStep);
      kread(B[0], kb);
      compute_step<1, 16, FUSED>(B, vb, first + k * kStep, hi, qB0, qB1, scale_log2, S, tl, lane, &pt);
      if (k + 1 >= n) break;
      load(B[0], kb, vb, first + (k + 2) * kStep);
      kread(A[0], ka);
      compute_step<1, 16, FUSED>(A, va, first + (k + 1) * kStep, hi, qB0, qB1, scale_log2, S, tl, lane, &pt);
    }
  }
  // The last request past the range still writes (zeros) into LDS when it returns: let it land
  // before the LDS is reused or the wave ends. s_waitcnt vmcnt(0).
  __builtin_amdgcn_s_waitcnt(0x0F70);
  float m = S.m;
  float lsum = sum_over_groups(S.lsum);
  f32x4 (&o)[4] = S.o;

  // Lane (r16, g) holds O^T[d = 16dt + 4g + i][head r16].
  if (NW == 1) {
    const bool mine = r16 < group;
    const int hq = kh * group + r16;
    if (ns == 1) {
      if (!mine) return;
      uint16_t *op = out + (int64_t)row * s_ob + (int64_t)hq * s_oh + 4 * g;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        st8(op + 16 * dt, u32x2{pack_bf16x2(o[dt][0] / lsum, o[dt][1] / lsum),
                                pack_bf16x2(o[dt][2] / lsum, o[dt][3] / lsum)});
      return;
    }
    if (!counters) {  // the combine kernel merges
      if (!mine) return;
      const int64_t pi = ((int64_t)row * nq + hq) * ns + sp;
      float *ap = acc_ws + pi * 64 + 4 * g;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) *reinterpret_cast<f32x4 *>(ap + 16 * dt) = o[dt];
      if (g == 0) {
        ml_ws[pi * 2] = m;
        ml_ws[pi * 2 + 1] = lsum;
      }
      return;
    }
    // In-kernel merge: the (row, kv head)'s partials [group heads][ns splits] as agent-coherent buffers.
    const int64_t p0i = ((int64_t)row * nq + (int64_t)kh * group) * ns;
    const rsrc_t acc_r = make_rsrc(acc_ws + p0i * 64, (uint32_t)(group * ns * 64 * 4));
    const rsrc_t ml_r = make_rsrc(ml_ws + p0i * 2, (uint32_t)(group * ns * 2 * 4));
    if (mine) {
      const uint32_t ao = (uint32_t)(((r16 * ns + sp) * 64 + 4 * g) * 4);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[dt]), acc_r, ao + 64u * dt, 0, kSC1);
      if (g == 0) {
        const uint32_t mo = (uint32_t)((r16 * ns + sp) * 2 * 4);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m), ml_r, mo, 0, kSC1);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(lsum), ml_r, mo + 4u, 0, kSC1);
      }
    }
    if (!last_arrival(counters + (int64_t)row * nkv + kh, ns)) return;
    if (mine) {
      f32x4 num[4];
      float den;
      merge_partials(acc_r, ml_r, r16, g, ns, scale_log2, num, den);
      uint16_t *op = out + (int64_t)row * s_ob + (int64_t)hq * s_oh + 4 * g;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        st8(op + 16 * dt, u32x2{pack_bf16x2(num[dt][0] / den, num[dt][1] / den),
                                pack_bf16x2(num[dt][2] / den, num[dt][3] / den)});
    }
    return;
  }

  // Merge the waves' partials through LDS (the V tiles are dead now: every wave's DMA has landed).
  __syncthreads();
  static_assert((32 + 16 * kOb) * 4 <= kVTile * 2, "merge buffer exceeds the V tiles");
  float *mb = reinterpret_cast<float *>(vbA);  // [NW][16]
  float *lb = mb + NW * 16;                     // [NW][16]
  float *ob = lb + NW * 16;                     // [NW][16 heads][64 dims]
  if (g == 0) {
    mb[w * 16 + r16] = m;
    lb[w * 16 + r16] = lsum;
  }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) *reinterpret_cast<f32x4 *>(ob + (w * 16 + r16) * kOb + 16 * dt + 4 * g) = o[dt];
  __syncthreads();
  const bool merge_here = ns > 1 && counters;
  const int64_t p0i = ((int64_t)row * nq + (int64_t)kh * group) * ns;
  const rsrc_t acc_r = make_rsrc(acc_ws + (merge_here ? p0i * 64 : 0), (uint32_t)(group * ns * 64 * 4));
  const rsrc_t ml_r = make_rsrc(ml_ws + (merge_here ? p0i * 2 : 0), (uint32_t)(group * ns * 2 * 4));
  for (int idx = threadIdx.x; idx < group * 64; idx += 64 * NW) {
    const int head = idx >> 6, d = idx & 63;
    float M = kNegInf;
#pragma unroll
    for (int v = 0; v < NW; ++v) M = fmaxf(M, mb[v * 16 + head]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const float mv = mb[v * 16 + head];
      const float wt = (mv == kNegInf) ? 0.f : fast_exp2((mv - M) * scale_log2);
      num += wt * ob[(v * 16 + head) * kOb + d];
      den += wt * lb[v * 16 + head];
    }
    const int hq = kh * group + head;
    if (ns == 1) {
      out[(int64_t)row * s_ob + (int64_t)hq * s_oh + d] = (uint16_t)(pack_bf16x2(num / den, 0.f) & 0xffffu);
    } else if (!merge_here) {
      const int64_t pi = ((int64_t)row * nq + hq) * ns + sp;
      acc_ws[pi * 64 + d] = num;
      if (d == 0) {
        ml_ws[pi * 2] = M;
        ml_ws[pi * 2 + 1] = den;
      }
    } else {
      const uint32_t e = (uint32_t)(head * ns + sp);
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(num), acc_r, (e * 64 + d) * 4, 0, kSC1);
      if (d == 0) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(M), ml_r, e * 8, 0, kSC1);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(den), ml_r, e * 8 + 4u, 0, kSC1);
      }
    }
  }
  if (!merge_here) return;
  // every thread's partial stores complete, then one arrival for the workgroup
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  __shared__ int last_flag;
  if (threadIdx.x < 64) {
    const bool last = last_arrival(counters + (int64_t)row * nkv + kh, ns);
    if (threadIdx.x == 0) last_flag = last ? 1 : 0;
  }
  __syncthreads();
  if (!last_flag) return;
  for (int idx = threadIdx.x; idx < group * 64; idx += 64 * NW) {
    const int head = idx >> 6, d = idx & 63;
    const float v = merge_partial_elem(acc_r, ml_r, head, d, ns, scale_log2);
    out[(int64_t)row * s_ob + (int64_t)(kh * group + head) * s_oh + d] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu);
  }
}

// One wave per (row, q head), lane = dim: merges the row's nsplit partials
// (fast_kernels.py:238-253).
__global__ __launch_bounds__(256) void k_decode_combine(const float *__restrict__ acc_ws,
                                                        const float *__restrict__ ml_ws,
                                                        uint16_t *__restrict__ out, int64_t s_ob, int64_t s_oh,
                                                        int b, int nq, int ns, float scale_log2) {
  const int pair = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pair >= b * nq) return;
  const int row = pair / nq, h = pair - row * nq, d = threadIdx.x & 63;
  const float *ml = ml_ws + (int64_t)pair * ns * 2;
  const float *acc = acc_ws + (int64_t)pair * ns * 64;
  // one pass with a running maximum (earlier weights rescaled when it grows), eight splits' loads in
  // flight at a time: the merge costs one memory round trip for up to eight splits
  constexpr int SB = 8;
  float M = kNegInf, num = 0.f, den = 0.f;
  for (int s0 = 0; s0 < ns; s0 += SB) {
    float mv[SB], lv[SB], av[SB];
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      const int sp = min(s0 + i, ns - 1);
      mv[i] = ml[2 * sp];
      lv[i] = ml[2 * sp + 1];
      av[i] = acc[sp * 64 + d];
    }
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      if (s0 + i >= ns) break;
      if (mv[i] == kNegInf) continue;  // an empty split adds nothing
      if (mv[i] > M) {
        const float sc = (M == kNegInf) ? 0.f : fast_exp2((M - mv[i]) * scale_log2);
        num *= sc;
        den *= sc;
        M = mv[i];
      }
      const float wt = fast_exp2((mv[i] - M) * scale_log2);
      num += wt * av[i];
      den += wt * lv[i];
    }
  }
  out[(int64_t)row * s_ob + (int64_t)h * s_oh + d] = (uint16_t)(pack_bf16x2(num / den, 0.f) & 0xffffu);
}

static inline bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int NW, bool FUSED>
static void launch_split(int ns, int nkv, int b, hipStream_t st, const uint16_t *q, int64_t s_qb, int64_t s_qh,
                         uint16_t *kc, uint16_t *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks, int cache_rows,
                         int cache_len, const int32_t *lens, const int32_t *rowmap, uint16_t *out, int64_t s_ob,
                         int64_t s_oh, float *acc_ws, float *ml_ws, int32_t *counters, int nq, int group,
                         float scale_log2, const StoreIn &si) {
  auto kern = k_decode_split<NW, FUSED>;
  hipLaunchKernelGGL(kern, dim3(ns, nkv, b), dim3(64 * NW), 0, st, q, s_qb, s_qh, kc, vc, s_kb, s_kh, s_ks,
                     cache_rows, cache_len, lens, rowmap, out, s_ob, s_oh, acc_ws, ml_ws, counters, nq, nkv, group,
                     ns, scale_log2, si);
}

// Body of a8_decode_attn and a8_store_decode_split (fused = si.qkv != nullptr: q is unused, the store's
// inputs are in si).
static int split_entry(const char *fn, const void *q, int64_t s_qb, int64_t s_qh, void *kc, void *vc, int64_t s_kb,
                       int64_t s_kh, int64_t s_ks, int cache_rows, int cache_len, const int32_t *lens,
                       const int32_t *rowmap, void *out, int64_t s_ob, int64_t s_oh, float *acc_ws, float *ml_ws,
                       int64_t ws_row_splits, int32_t *counters, int64_t n_counters, int b, int nq, int nkv, int hd,
                       int nsplit, int waves, float scale, int phases, const StoreIn &si, void *stream) {
  const bool fused = si.qkv != nullptr;
  if (hd != 64 && (fused || hd != 128))
    return set_error(A8_EUNSUP, "%s: head_dim %d not supported (64; 128 through the unfused call)", fn, hd);
  if (b < 0 || nq <= 0 || nkv <= 0 || nq % nkv || cache_rows < 0 || cache_len < 0 || nsplit < 1 || b > 65535)
    return set_error(A8_EINVAL, "%s: bad sizes b=%d nq=%d nkv=%d nsplit=%d", fn, b, nq, nkv, nsplit);
  const int group = nq / nkv;
  if (group > (fused ? kLaneK : 16))
    return set_error(A8_EUNSUP, "%s: GQA group %d > %d not supported", fn, group, fused ? kLaneK : 16);
  if (waves != 1 && waves != 2 && waves != 4 && waves != 8)
    return set_error(A8_EINVAL, "%s: waves must be 1, 2, 4 or 8 (got %d)", fn, waves);
  if (b == 0) return 0;
  if ((!fused && !q) || !kc || !vc || !lens || !out) return set_error(A8_EINVAL, "%s: null pointer", fn);
  if (nsplit > 1 && (!acc_ws || !ml_ws || (int64_t)b * nsplit > ws_row_splits))
    return set_error(A8_EWSPACE, "%s: workspace holds %lld row-splits, need b*nsplit = %lld", fn,
                     (long long)ws_row_splits, (long long)b * nsplit);
  if (s_ks != hd)
    return set_error(A8_EUNSUP, "%s: cache positions must be contiguous rows (s_ks %lld)", fn, (long long)s_ks);
  if (counters && (int64_t)b * nkv > n_counters)
    return set_error(A8_EWSPACE, "%s: %lld counters, need b*nkv = %lld", fn, (long long)n_counters,
                     (long long)b * nkv);
  if (counters && nsplit > 1 && (int64_t)group * nsplit * 64 * 4 > (int64_t)UINT32_MAX)
    return set_error(A8_EUNSUP, "%s: %d splits too many for the in-kernel merge", fn, nsplit);
  if (counters && nsplit > 1 && (phases & 1) == 0)
    return set_error(A8_EINVAL, "%s: with counters the merge is part of the split kernel (phases bit 0)", fn);
  if ((!fused && !al16(q)) || !al16(kc) || !al16(vc) || !al16(out) || (nsplit > 1 && !al16(acc_ws)) ||
      ((fused ? 0 : (s_qb | s_qh)) | s_kb | s_kh | s_ks | s_ob | s_oh) & 7)
    return set_error(A8_EALIGN, "%s: pointers must be 16-byte aligned and strides multiples of 8", fn);
  if (hd != 64)  // the generic-head kernel (one launch, no workspace)
    return attn_cols_decode(fn, q, s_qb, s_qh, kc, vc, s_kb, s_kh, cache_rows, cache_len, lens, rowmap, out, s_ob,
                            s_oh, b, nq, nkv, hd, scale, (hipStream_t)stream);
  const hipStream_t st = (hipStream_t)stream;
  const float sl2 = scale * kLog2e;
  const auto *qq = (const uint16_t *)q;
  auto *kk = (uint16_t *)kc;
  auto *vv = (uint16_t *)vc;
  auto *oo = (uint16_t *)out;
  if (phases & 1) {
#define A8_SPLIT_ARGS nsplit, nkv, b, st, qq, s_qb, s_qh, kk, vv, s_kb, s_kh, s_ks, cache_rows, cache_len, lens, \
                      rowmap, oo, s_ob, s_oh, acc_ws, ml_ws, counters, nq, group, sl2, si
    switch (waves * 2 + (fused ? 1 : 0)) {
      case 2: launch_split<1, false>(A8_SPLIT_ARGS); break;
      case 3: launch_split<1, true>(A8_SPLIT_ARGS); break;
      case 4: launch_split<2, false>(A8_SPLIT_ARGS); break;
      case 5: launch_split<2, true>(A8_SPLIT_ARGS); break;
      case 8: launch_split<4, false>(A8_SPLIT_ARGS); break;
      case 9: launch_split<4, true>(A8_SPLIT_ARGS); break;
      case 17: launch_split<8, true>(A8_SPLIT_ARGS); break;
      default: launch_split<8, false>(A8_SPLIT_ARGS); break;
    }
#undef A8_SPLIT_ARGS
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  if ((phases & 2) && nsplit > 1 && !counters) {
    const unsigned grid = (unsigned)(((int64_t)b * nq + 3) / 4);
    hipLaunchKernelGGL(k_decode_combine, dim3(grid), dim3(256), 0, st, acc_ws, ml_ws, oo, s_ob, s_oh, b, nq,
                       nsplit, sl2);
    return (int)hipGetLastError();
  }
  return 0;
}

}  // namespace a8

extern "C" int a8_decode_attn(const void *q, int64_t s_qb, int64_t s_qh,
                              const void *kc, const void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                              int cache_rows, int cache_len,
                              const int32_t *lens, const int32_t *rowmap,
                              void *out, int64_t s_ob, int64_t s_oh,
                              float *acc_ws, float *ml_ws, int64_t ws_row_splits,
                              int32_t *counters, int64_t n_counters,
                              int b, int nq, int nkv, int hd, int nsplit, int waves, float scale,
                              int phases, void *stream) {
  using namespace a8;
  const StoreIn none{};
  return split_entry("decode_attn", q, s_qb, s_qh, const_cast<void *>(kc), const_cast<void *>(vc), s_kb, s_kh, s_ks,
                     cache_rows, cache_len, lens, rowmap, out, s_ob, s_oh, acc_ws, ml_ws, ws_row_splits, counters,
                     n_counters, b, nq, nkv, hd, nsplit, waves, scale, phases, none, stream);
}

extern "C" int a8_store_decode_split(const void *qkv, int64_t s_qkv, const void *bias,
                                     const void *cos_tab, const void *sin_tab, int64_t s_cs, int n_tab,
                                     const int32_t *pos, const int32_t *slot,
                                     void *qo, int64_t s_qo_r, int64_t s_qo_h,
                                     void *kc, void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                                     int cache_rows, int cache_len, const int32_t *lens, const int32_t *rowmap,
                                     void *out, int64_t s_ob, int64_t s_oh,
                                     float *acc_ws, float *ml_ws, int64_t ws_row_splits,
                                     int32_t *counters, int64_t n_counters,
                                     int b, int nq, int nkv, int hd, int ring, int nsplit, int waves, float scale,
                                     int phases, void *stream) {
  using namespace a8;
  if (ring <= 0 || n_tab < 0) return set_error(A8_EINVAL, "store_decode_split: bad ring %d / n_tab %d", ring, n_tab);
  if (b > 0 && (!qkv || !cos_tab || !sin_tab || !pos || !slot))
    return set_error(A8_EINVAL, "store_decode_split: null pointer");
  if (b > 0 && (!al16(qkv) || !al16(cos_tab) || !al16(sin_tab) || (bias && !al16(bias)) || (qo && !al16(qo)) ||
                (s_qkv | s_cs | (qo ? (s_qo_r | s_qo_h) : 0)) & 7))
    return set_error(A8_EALIGN, "store_decode_split: pointers must be 16-byte aligned and strides multiples of 8");
  if (b > 0 && (phases & 1) == 0)  // the store is part of the split kernel
    return set_error(A8_EINVAL, "store_decode_split: phases must include the split kernel (bit 0)");
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
  return split_entry("store_decode_split", nullptr, 0, 0, kc, vc, s_kb, s_kh, s_ks, cache_rows, cache_len, lens,
                     rowmap, out, s_ob, s_oh, acc_ws, ml_ws, ws_row_splits, counters, n_counters, b, nq, nkv, hd,
                     nsplit, waves, scale, phases, si, stream);
}

// Launch-shape policy (measured on MI355X at 192 slots x 2048 keys: one split of 4 waves per
// (row, kv head) streams the cache at ~42 us/layer; extra splits save ~3 us in the split kernel but
// the combine launch costs 3-4 us). So: one split whenever the rows x kv heads already give every
// compute unit a workgroup, and more splits only when they do not (small batches, long caches), up
// to about two workgroups per compute unit and at least two 64-key tiles per wave.
extern "C" int a8_decode_choose(int b, int nkv, int cache_len, int nsplit_req, int nsplit_max,
                                int64_t cap_row_splits, int n_cu, int *nsplit_out, int *waves_out) {
  using namespace a8;
  if (b < 1 || nkv < 1 || cache_len < 0 || n_cu < 1 || !nsplit_out || !waves_out)
    return set_error(A8_EINVAL, "decode_choose: bad arguments b=%d nkv=%d n_cu=%d", b, nkv, n_cu);
  const int tiles = cache_len > 0 ? (cache_len + 63) / 64 : 1;
  const int nw = tiles >= 8 ? 4 : tiles >= 4 ? 2 : 1;
  const int64_t units = (int64_t)b * nkv;
  int64_t ns = 1;
  if (units < n_cu) {
    ns = (2 * (int64_t)n_cu + units - 1) / units;
    const int64_t by_tiles = tiles / (2 * nw);  // keep >= 2 tiles per wave
    if (ns > by_tiles) ns = by_tiles;
  }
  if (ns < nsplit_req) ns = nsplit_req;
  if (nsplit_max >= 1 && ns > nsplit_max) ns = nsplit_max;
  if (ns > tiles) ns = tiles;
  if (cap_row_splits >= 1 && ns > cap_row_splits / b) ns = cap_row_splits / b;
  if (ns < 1) ns = 1;
  // once the splits give every compute unit a workgroup, one wave per split: no merge across waves
  // (measured at 64 ragged rows over a 4096-key cache: 4 x 1 waves 15.1 us/layer against 4 x 4 15.8)
  const int nw_out = (ns > 1 && units * ns >= n_cu) ? 1 : nw;
  *nsplit_out = (int)ns;
  *waves_out = nw_out;
  return 0;
}

// ---- a8_decode_attn_noalloc: the split + combine launch with its partials in a fixed device array ----
namespace a8 {

// The split partials (acc [b, nq, nsplit, 64] then ml [b, nq, nsplit, 2], fp32) of a8_decode_attn_noalloc.
// Every GPU the library runs on holds its own copy from module load until the process ends. Host code never
// uses the name (on the host it is only a stand-in for the symbol): it uses the address that
// hipGetSymbolAddress returns for the current device, kept per device in g_scratch_dev.
constexpr int64_t kScratchFloats = A8_NOALLOC_SCRATCH_BYTES / 4;
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
static float *g_scratch_dev[kMaxDevices];
static std::mutex g_scratch_mu;

// The copy of `scratch` on the device that `stream` belongs to (the current device for the null stream),
// looked up once per device with that device current, or nullptr with the error recorded.
static float *scratch_for_stream(const char *fn, hipStream_t stream) {
  int cur = -1, dev = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) {
    set_error(A8_EINVAL, "%s: hipGetDevice failed (%d)", fn, (int)e);
    return nullptr;
  }
  dev = cur;
  if (stream) {
    e = hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess) {
      set_error(A8_EINVAL, "%s: hipStreamGetDevice failed (%d)", fn, (int)e);
      return nullptr;
    }
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error(A8_EUNSUP, "%s: device %d beyond the %d supported", fn, dev, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    // hipGetSymbolAddress answers for the current device: make the stream's device current for the lookup
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) {
      set_error(A8_EINVAL, "%s: hipSetDevice(%d) failed (%d)", fn, dev, (int)e);
      return nullptr;
    }
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) hipSetDevice(cur);
    if (e != hipSuccess || !p) {
      set_error(A8_EINVAL, "%s: hipGetSymbolAddress(scratch) failed on device %d (%d)", fn, dev, (int)e);
      return nullptr;
    }
    g_scratch_dev[dev] = static_cast<float *>(p);
  }
  return g_scratch_dev[dev];
}

}  // namespace a8

extern "C" int a8_decode_attn_noalloc(const void *q, int64_t s_qb, int64_t s_qh,
                                      const void *kc, const void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                                      int cache_rows, int cache_len,
                                      const int32_t *lens, const int32_t *rowmap,
                                      void *out, int64_t s_ob, int64_t s_oh,
                                      int b, int nq, int nkv, int hd, int nsplit, int waves, float scale,
                                      void *stream) {
  using namespace a8;
  const char *fn = "decode_attn_noalloc";
  if (b < 0 || nq <= 0 || hd <= 0 || nsplit < 1)
    return set_error(A8_EINVAL, "%s: bad sizes b=%d nq=%d hd=%d nsplit=%d", fn, b, nq, hd, nsplit);
  if (b == 0) return 0;
  float *acc = nullptr, *ml = nullptr;
  int64_t row_splits = 0;
  if (nsplit > 1 && hd == 64) {  // head_dim 128 takes the generic-head kernel, which uses no partials
    // every (row, head, split) partial the combine reads is written by the split kernel first: nothing in
    // the array has to start at zero
    const int64_t parts = (int64_t)b * nq * nsplit;
    const int64_t need = parts * ((int64_t)hd + 2);
    if (need > kScratchFloats)
      return set_error(A8_EWSPACE, "%s: b*nq*nsplit*(hd+2) = %lld floats exceed the fixed %lld-float scratch "
                       "(8 MiB); use a8_decode_attn with a caller workspace", fn, (long long)need,
                       (long long)kScratchFloats);
    float *base = scratch_for_stream(fn, (hipStream_t)stream);
    if (!base) return A8_EINVAL;
    acc = base;
    ml = base + parts * hd;  // parts * hd floats in: a multiple of 64 floats, 256-byte aligned
    row_splits = (int64_t)b * nsplit;
  }
  const StoreIn none{};
  return split_entry(fn, q, s_qb, s_qh, const_cast<void *>(kc), const_cast<void *>(vc), s_kb, s_kh, s_ks,
                     cache_rows, cache_len, lens, rowmap, out, s_ob, s_oh, acc, ml, row_splits, nullptr, 0, b, nq,
                     nkv, hd, hd == 64 ? nsplit : 1, waves, scale, 3, none, stream);
}
