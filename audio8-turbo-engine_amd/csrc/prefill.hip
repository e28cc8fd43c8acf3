// Packed variable-length causal prefill attention over cache rows (a8_prefill_attn).
//
// Semantics follow serve/fast_kernels.py:296-358 (_prefill_attn_kernel / prefill_attention): a
// block of <= 64 packed query rows [q0, q0+n) of one request sits at positions [p0, p0+n) of cache
// row `slot`; each row attends keys [0, p0+n) of that row with key <= its position (the cached
// voice prefix [0, p0) plus the causal part of the new tokens), online softmax in fp32, bf16
// softmax weights in P.V, out = bf16(acc / l).
//
// MI355X design (compute-heavy: ~325 FLOP per compulsory byte, so both products run on MFMA):
//   * One workgroup = one query block x one kv head; its waves are the kv head's q heads (GQA
//     group, up to 8 per workgroup), so each K/V tile is staged in LDS once and read by every head.
//   * K tile [64 keys][64 d] is staged row-major; the V tile is staged transposed (V^T[d][key]) by
//     8-key x 16-byte register transposes, so both products read 128-bit MFMA operands from LDS.
//   * Per wave: S^T = K . Q^T (v_mfma_f32_16x16x32_bf16, 64 keys x 64 query rows per tile), online
//     softmax per query column, O^T += V^T . P^T with the S^T C-layout reused as the P^T B operand
//     (key rows permuted within 32-key chunks, as in the decode kernel).
#include "a8_common.h"

namespace a8 {

constexpr int kPfRow = 72;    // LDS row: 64 bf16 + 8 pad (144 B)
constexpr int kPfMaxHW = 8;   // q heads (waves) per workgroup

__global__ __launch_bounds__(64 * kPfMaxHW) void k_prefill(
    const uint16_t *__restrict__ q, int64_t s_qr, int64_t s_qh, int R,
    const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
    int cache_rows, int cache_len, uint16_t *__restrict__ out, int64_t s_or, int64_t s_oh,
    const int32_t *__restrict__ bq0, const int32_t *__restrict__ bn, const int32_t *__restrict__ bslot,
    const int32_t *__restrict__ bpos0, int group, int hsplit, int hpw, float scale_log2) {
  __shared__ __attribute__((aligned(16))) uint16_t ks[64 * kPfRow];
  __shared__ __attribute__((aligned(16))) uint16_t vt[64 * kPfRow];
  const int blk = blockIdx.x;
  const int kh = blockIdx.y / hsplit, hs = blockIdx.y - kh * hsplit;
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int lane = tid & 63, w = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;

  // Block metadata is uniform over the workgroup, so early exits happen before any barrier.
  const int n = bn[blk];
  if (n <= 0) return;  // graph-mode padding block
  const int q0 = bq0[blk], p0 = bpos0[blk];
  const int64_t sl = bslot[blk];
  if (sl < 0 || sl >= cache_rows || p0 < 0 || q0 < 0 || q0 >= R) return;
  const int nv = min(min(n, 64), R - q0);  // valid query rows
  const int hi = min(p0 + n, cache_len);   // keys [0, hi)
  if (hi <= 0) return;

  const int gi = hs * hpw + w;  // head index within the group
  const bool active = gi < group;
  const int h = kh * group + gi;

  // Q^T operands (B of S^T = K.Q^T): column r16 <-> query row 16qt + r16, slot (g, j) <-> dim
  // 8g+j (hh = 0) and 32+8g+j (hh = 1).
  u32x4 qB[4][2];
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    const int mrow = 16 * qt + r16;
    if (active && mrow < nv) {
      const uint16_t *qp = q + (int64_t)(q0 + mrow) * s_qr + (int64_t)h * s_qh + 8 * g;
      qB[qt][0] = ld16(qp);
      qB[qt][1] = ld16(qp + 32);
    } else {
      qB[qt][0] = u32x4{0u, 0u, 0u, 0u};
      qB[qt][1] = u32x4{0u, 0u, 0u, 0u};
    }
  }
  float mrun[4], lrun[4];
  f32x4 o[4][4];  // [dt][qt]: O^T rows d = 16dt + 4g + i, column = query row 16qt + r16
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    mrun[qt] = kNegInf;
    lrun[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const uint16_t *kb = kc + sl * s_kb + (int64_t)kh * s_kh;
  const uint16_t *vb = vc + sl * s_kb + (int64_t)kh * s_kh;

  for (int kt0 = 0; kt0 < hi; kt0 += 64) {
    const int last = hi - 1;
    // ---- stage K[key][d] and V^T[d][key] for keys kt0..kt0+63 (clamped to the range) ----
    for (int i = tid; i < 512; i += nthr) {
      const int kr = i >> 3, ch = i & 7;
      const int key = min(kt0 + kr, last);
      st16(ks + kr * kPfRow + 8 * ch, ld16(kb + (int64_t)key * s_ks + 8 * ch));
    }
    for (int u = tid; u < 64; u += nthr) {
      const int kg = u >> 3, dc = u & 7;
      u32x4 vr[8], vtr[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) vr[j] = ld16(vb + (int64_t)min(kt0 + 8 * kg + j, last) * s_ks + 8 * dc);
      transpose8x8_bf16(vr, vtr);
#pragma unroll
      for (int dd = 0; dd < 8; ++dd) st16(vt + (8 * dc + dd) * kPfRow + 8 * kg, vtr[dd]);
    }
    __syncthreads();

    if (active) {
      // ---- S^T = K.Q^T; tile (c, t) row 4g+i <-> key kt0 + 32c + 8g + 4t + i ----
      f32x4 s[2][2][4];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const uint16_t *kr = ks + (32 * c + 8 * (r16 >> 2) + 4 * t + (r16 & 3)) * kPfRow + 8 * g;
          const u32x4 ka0 = ld16(kr), ka1 = ld16(kr + 32);
#pragma unroll
          for (int qt = 0; qt < 4; ++qt) {
            f32x4 a = mfma16x16x32(ka0, qB[qt][0], f32x4{0.f, 0.f, 0.f, 0.f});
            s[c][t][qt] = mfma16x16x32(ka1, qB[qt][1], a);
          }
        }
      // ---- causal mask + online softmax per query column ----
      u32x4 pB[2][4];
      float alpha[4];
#pragma unroll
      for (int qt = 0; qt < 4; ++qt) {
        const int lim = min(p0 + 16 * qt + r16, last);  // keys <= query position (and < hi)
        float mt = kNegInf;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int key = kt0 + 32 * c + 8 * g + 4 * t + i;
              const float v = key <= lim ? s[c][t][qt][i] * scale_log2 : kNegInf;
              s[c][t][qt][i] = v;
              mt = fmaxf(mt, v);
            }
        mt = max_over_groups(mt);
        const float mn = fmaxf(mrun[qt], mt);
        // mn stays -inf only for a column with no key yet (a padding row): keep it inert.
        const float mref = mn == kNegInf ? 0.f : mn;
        alpha[qt] = (mrun[qt] == kNegInf) ? 0.f : fast_exp2(mrun[qt] - mref);
        float ps = 0.f;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              p[i] = fast_exp2(s[c][t][qt][i] - mref);
              ps += p[i];
            }
            pB[c][qt][2 * t] = pack_bf16x2(p[0], p[1]);
            pB[c][qt][2 * t + 1] = pack_bf16x2(p[2], p[3]);
          }
        lrun[qt] = lrun[qt] * alpha[qt] + ps;
        mrun[qt] = mn;
      }
      // ---- O^T += V^T . P^T ----
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
        for (int qt = 0; qt < 4; ++qt) o[dt][qt] *= alpha[qt];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const u32x4 vA = ld16(vt + (16 * dt + r16) * kPfRow + 32 * c + 8 * g);
#pragma unroll
          for (int qt = 0; qt < 4; ++qt) o[dt][qt] = mfma16x16x32(vA, pB[c][qt], o[dt][qt]);
        }
      }
    }
    __syncthreads();
  }

  if (!active) return;
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    const float l = sum_over_groups(lrun[qt]);
    const int mrow = 16 * qt + r16;
    if (mrow >= nv) continue;
    uint16_t *op = out + (int64_t)(q0 + mrow) * s_or + (int64_t)h * s_oh + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      st8(op + 16 * dt, u32x2{pack_bf16x2(o[dt][qt][0] / l, o[dt][qt][1] / l),
                              pack_bf16x2(o[dt][qt][2] / l, o[dt][qt][3] / l)});
  }
}

static inline bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace a8

extern "C" int a8_prefill_attn(const void *q, int64_t s_qr, int64_t s_qh, int R,
                               const void *kc, const void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                               int cache_rows, int cache_len,
                               void *out, int64_t s_or, int64_t s_oh,
                               const int32_t *bq0, const int32_t *bn, const int32_t *bslot,
                               const int32_t *bpos0, int nblk, int bm,
                               int nq, int group, int hd, float scale, void *stream) {
  using namespace a8;
  if (hd != 64) return set_error(A8_EUNSUP, "prefill_attn: head_dim %d not supported (64 only)", hd);
  if (bm != 64) return set_error(A8_EUNSUP, "prefill_attn: block size %d not supported (64 only)", bm);
  if (nblk < 0 || R < 0 || nq <= 0 || group <= 0 || nq % group || cache_rows < 0 || cache_len < 0)
    return set_error(A8_EINVAL, "prefill_attn: bad sizes nblk=%d R=%d nq=%d group=%d", nblk, R, nq, group);
  if (nblk == 0 || R == 0) return 0;
  if (!q || !kc || !vc || !out || !bq0 || !bn || !bslot || !bpos0)
    return set_error(A8_EINVAL, "prefill_attn: null pointer");
  if (!al16(q) || !al16(kc) || !al16(vc) || !al16(out) || (s_qr | s_qh | s_kb | s_kh | s_ks | s_or | s_oh) & 7)
    return set_error(A8_EALIGN, "prefill_attn: pointers must be 16-byte aligned and strides multiples of 8");
  const int nkv = nq / group;
  const int hpw = group < kPfMaxHW ? group : kPfMaxHW;
  const int hsplit = (group + hpw - 1) / hpw;
  if ((int64_t)nkv * hsplit > 65535) return set_error(A8_EUNSUP, "prefill_attn: too many heads");
  hipLaunchKernelGGL(k_prefill, dim3(nblk, nkv * hsplit), dim3(64 * hpw), 0, (hipStream_t)stream,
                     (const uint16_t *)q, s_qr, s_qh, R, (const uint16_t *)kc, (const uint16_t *)vc, s_kb, s_kh,
                     s_ks, cache_rows, cache_len, (uint16_t *)out, s_or, s_oh, bq0, bn, bslot, bpos0, group, hsplit,
                     hpw, scale * kLog2e);
  return (int)hipGetLastError();
}
