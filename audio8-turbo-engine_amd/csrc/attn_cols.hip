// Decode attention for head dimensions other than 64 (head_dim 128): a8_decode_attn* through one kernel, for
// the reference's generic-HD decode kernels (serve/fast_kernels.py:190-290: HD is a compile-time constant
// there, any power of two). The head_dim-128 packed prefill is prefill128.hip.
//
// One wave computes up to 16 attention columns that share a cache row and a kv head; column j (lane r16 = j of
// each 16-lane group) is q head kh * group + j of one query row, which attends keys [0, L) of the cache row
// (L = lens), online softmax in fp32 (exp2 with the scale folded in, the weights rounded to bf16 for P.V as in
// the reference, the row sum of the fp32 weights), out = bf16(acc / l).
//
// Per 64-key tile, with the MFMA layouts of the head_dim-64 kernels (v_mfma_f32_16x16x32_bf16):
//   * S^T = K.Q^T: tile (c, t) rows 4g+i <-> key t0 + 32c + 8g + 4t + i; the K operand (lane (g, r16): key
//     t0 + 32c + 8(r16/4) + 4t + r16%4, dims 32s + 8g..+7) comes straight from the cache with 16-byte buffer
//     loads (keys past the wave's largest L read as zeros), HD/32 products per (c, t);
//   * O^T += V^T.P^T: the S^T C layout is the P^T operand; V goes by DMA (buffer_load ... lds) into a
//     wave-private LDS tile, row r's 16-byte chunks permuted by chunk ^= 2 (r & 3) (the permutation goes into
//     the DMA's source offsets), so the transposing reads of four consecutive rows hit distinct banks; it is
//     read as V^T by ds_read_b64_tr_b16, HD/16 row blocks of 16 dims.
// One wave per workgroup and column group, two tile buffers: the next tile's K / V requests in flight while a
// tile is computed (four waves with one buffer measured 105.8 us per layer at 192 rows x 2048 keys, 0.48 of
// HBM; this 73.4 us, 0.69).
#include "decode_tile.h"

namespace a8 {
namespace {


template <int HD>
__global__ __launch_bounds__(64) void k_attn_cols(
    const uint16_t *__restrict__ q, int64_t s_qr, int64_t s_qh,
    const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc, int64_t s_kb, int64_t s_kh,
    int cache_rows, int cache_len, uint16_t *__restrict__ out, int64_t s_or, int64_t s_oh,
    const int32_t *__restrict__ lens, const int32_t *__restrict__ rowmap, int ngroups, int nkv, int group,
    float sl2) {
  static_assert(HD % 32 == 0 && HD <= 128, "head dimension");
  constexpr int KS = HD / 32;   // reduction slices of S^T
  constexpr int DT = HD / 16;   // 16-dim row blocks of O^T
  constexpr int PITCH = HD * 2;  // bytes per key row of the LDS V tile
  constexpr int NCH = HD / 8;    // 16-byte chunks per key row
  // the two V tile buffers (separate arrays)
  __shared__ __attribute__((aligned(16))) char vbA[64 * PITCH];
  __shared__ __attribute__((aligned(16))) char vbB[64 * PITCH];
  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15, g = lane >> 4;
  const int gw = blockIdx.x;
  if (gw >= ngroups) return;

  // group gw = (row b, kv head kh); column j = q head kh * group + j of row b
  const int b = gw / nkv;
  const int kh = gw - b * nkv;
  const int crow = rowmap ? rowmap[b] : b;
  const int L = min(max(lens[b], 0), cache_len);
  if (crow < 0 || crow >= cache_rows) return;
  const bool valid = r16 < group;  // this lane's column exists
  const int head = kh * group + r16;
  const int Lc = valid ? L : 0;    // this column's key count

  // Q^T operands: column r16, dims 32s + 8g..+7 (zeros for a missing column)
  u32x4 qb[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) qb[s] = u32x4{0u, 0u, 0u, 0u};
  if (valid) {  // (a missing column's address may lie past q)
    const uint16_t *qp = q + (int64_t)b * s_qr + (int64_t)head * s_qh + 8 * g;
#pragma unroll
    for (int s = 0; s < KS; ++s) qb[s] = ld16(qp + 32 * s);
  }
  // K / V of the cache row and kv head as buffers over keys [0, L): rows past it read as zeros
  const int64_t cb = (int64_t)crow * s_kb + (int64_t)kh * s_kh;
  constexpr uint32_t kRowB = HD * 2;
  const rsrc_t kr = make_rsrc(kc + cb, (uint32_t)L * kRowB);
  const rsrc_t vr = make_rsrc(vc + cb, (uint32_t)L * kRowB);
  // K operand rows of this lane: key 32c + 8(r16/4) + 4t + r16%4 of the tile
  const uint32_t krow = (uint32_t)(8 * (r16 >> 2) + (r16 & 3));
  // V DMA: instruction i writes rows (16 i + lane) / NCH.., lane l's 16 bytes to LDS chunk l % NCH of its row,
  // from source chunk (l % NCH) ^ 2 (row & 3)
  constexpr int VDMA = 64 * NCH / 64;  // instructions per tile
  static_assert(64 % NCH == 0, "whole rows per DMA instruction");
  const uint32_t vrow = (uint32_t)(lane / NCH), vch = (uint32_t)(lane % NCH);
  const uint32_t vsrc = vrow * PITCH + ((vch ^ (2u * (vrow & 3u))) << 4);
  // V^T reads: lane i of a 16-lane group points at row r0 + i/4 (r0 = 32c + 8g, + 4), dims 16dt + 4(i%4),
  // found in LDS chunk (2dt + (i%4)/2) ^ 2 ((i/4) & 3)
  const uint32_t vrr = (uint32_t)(r16 >> 2), vperm = 2u * (vrr & 3u), vhalf = (uint32_t)(r16 & 1) * 8u;
  const uint32_t vc0 = (uint32_t)((r16 & 3) >> 1);

  float m = kNegInf, lsum = 0.f;
  f32x4 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Two tile buffers (V in LDS, K in registers), the next tile's loads in flight while one is computed; a
  // request past L reads zeros without memory traffic.
  u32x4 kA[2][2][KS], kB[2][2][KS];
  auto load = [&](u32x4 (&ka)[2][2][KS], char *vtile, int t0) __attribute__((always_inline)) {
    // every earlier read of this buffer done before its DMA can land
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
#pragma unroll
    for (int i = 0; i < VDMA; ++i)
      bld16_lds<0>(vr, vtile + i * 1024, (uint32_t)t0 * kRowB + (uint32_t)i * 1024u + vsrc, 0u);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int s = 0; s < KS; ++s)
          ka[c][t][s] = bld16(kr, ((uint32_t)t0 + 32u * c + krow + 4u * t) * kRowB + (uint32_t)(32 * s + 8 * g) * 2u);
  };
  // consumes the tile at t0 (K in ka, V in vtile); the V reads wait for its DMA: after it went out, its own
  // 4 KS K loads and the next tile's VDMA + 4 KS requests
  auto tile = [&](const u32x4 (&ka)[2][2][KS], const char *vtile, int t0) __attribute__((always_inline)) {
    // scores, masked where the tile reaches past the key count (and for a missing column)
    f32x4 sc[2][2];
    float mt = kNegInf;
    const bool mask = t0 + 64 > L || !valid;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) a = mfma16x16x32(ka[c][t][s], qb[s], a);
        if (mask) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (t0 + 32 * c + 8 * g + 4 * t + i >= Lc) a[i] = kNegInf;
        }
        mt = fmaxf(mt, fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3])));
        sc[c][t] = a;
      }
    mt = max_over_groups(mt);
    const float mn = fmaxf(m, mt);
    const float mc = mn == kNegInf ? 0.f : mn * sl2;  // a column with no key yet stays inert
    const float alpha = m == kNegInf ? 0.f : fast_exp2(__builtin_fmaf(m, sl2, -mc));
    float ps = 0.f;
    u32x4 pB[2];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[i] = fast_exp2(__builtin_fmaf(sc[c][t][i], sl2, -mc));
          ps += p[i];
        }
        pB[c][2 * t] = pack_bf16x2(p[0], p[1]);
        pB[c][2 * t + 1] = pack_bf16x2(p[2], p[3]);
      }
    lsum = lsum * alpha + ps;
    m = mn;
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
    }
    wait_vmcnt<8 * KS + VDMA>();  // the V tile has landed
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const char *p = vtile + (32 * c + 8 * g + vrr) * PITCH + ((((uint32_t)(2 * dt) + vc0) ^ vperm) << 4) + vhalf;
        const u32x2 lo = lds_tr16(p), hi2 = lds_tr16(p + 4 * PITCH);
        o[dt] = mfma16x16x32(u32x4{lo[0], lo[1], hi2[0], hi2[1]}, pB[c], o[dt]);
      }
  };
  load(kA, vbA, 0);
  for (int t0 = 0; t0 < L; t0 += 128) {
    load(kB, vbB, t0 + 64);
    tile(kA, vbA, t0);
    if (t0 + 64 >= L) break;
    load(kA, vbA, t0 + 128);
    tile(kB, vbB, t0 + 64);
  }
  // the request past the last tile still writes (zeros) into LDS: let it land before the wave ends
  wait_vmcnt<0>();

  // l = 0 (no key, decode lens = 0) gives 0 * inf = NaN, like the reference's 0 / 0
  const float rl = __builtin_amdgcn_rcpf(sum_over_groups(lsum));
  if (!valid) return;
  uint16_t *op = out + (int64_t)b * s_or + (int64_t)head * s_oh + 4 * g;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
    st8(op + 16 * dt, u32x2{pack_bf16x2(o[dt][0] * rl, o[dt][1] * rl), pack_bf16x2(o[dt][2] * rl, o[dt][3] * rl)});
}

}  // namespace

// Decode of b rows (a8_decode_attn / _stream / _flat / _noalloc for head_dim 128): q [b, nq, HD] (strides
// s_qb, s_qh), caches [rows, nkv, S, HD] with contiguous positions, lens / rowmap as the decode entry points.
int attn_cols_decode(const char *fn, const void *q, int64_t s_qb, int64_t s_qh, const void *kc, const void *vc,
                     int64_t s_kb, int64_t s_kh, int cache_rows, int cache_len, const int32_t *lens,
                     const int32_t *rowmap, void *out, int64_t s_ob, int64_t s_oh, int b, int nq, int nkv, int hd,
                     float scale, hipStream_t stream) {
  if (hd != 128) return set_error(A8_EUNSUP, "%s: head_dim %d not supported (64 or 128)", fn, hd);
  const int group = nq / nkv;
  if (group > 16) return set_error(A8_EUNSUP, "%s: GQA group %d > 16 not supported", fn, group);
  const int64_t ngroups = (int64_t)b * nkv;
  if (ngroups == 0) return 0;
  if (ngroups > INT32_MAX / 2) return set_error(A8_EUNSUP, "%s: %d rows x %d kv heads too many", fn, b, nkv);
  if ((int64_t)cache_len * hd * 2 >= ((int64_t)1 << 32))
    return set_error(A8_EUNSUP, "%s: cache of %d positions too long for 32-bit offsets", fn, cache_len);
  hipLaunchKernelGGL((k_attn_cols<128>), dim3((unsigned)ngroups), dim3(64), 0, stream, (const uint16_t *)q, s_qb,
                     s_qh, (const uint16_t *)kc, (const uint16_t *)vc, s_kb, s_kh, cache_rows, cache_len,
                     (uint16_t *)out, s_ob, s_oh, lens, rowmap, (int)ngroups, nkv, group, scale * kLog2e);
  return (int)hipGetLastError();
}

}  // namespace a8
