// qkv bias + rotate_half RoPE arithmetic of serve/fast_kernels.py:139-187, per partner pair of 16-byte
// chunks (dims 8c..8c+7 and HD/2+8c..HD/2+8c+7 of one head, HD the head dimension), shared by the store
// kernel (store.hip) and the fused store + decode paths (decode_stream.hip, decode_rows.hip), so both
// produce the same bits:
//   x = f32(qkv) + f32(bias)
//   q/k: o[d] = bf16(x[d] * cos[d] + sign(d) * x[(d + HD/2) % HD] * sin[d]),  sign = -1 for d < HD/2
//   v:   o[d] = bf16(x[d])
// with two roundings for the products and one for the sum (no contraction) and a torch-exact
// round-to-nearest-even narrowing.
#pragma once

#include "a8_common.h"

namespace a8 {

// x of the pair: wlo / whi are the qkv chunks, blo / bhi the bias chunks (ignored when has_bias is false).
__device__ __forceinline__ void rope_x(u32x4 wlo, u32x4 whi, u32x4 blo, u32x4 bhi, bool has_bias, float (&xl)[8],
                                       float (&xh)[8]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    xl[2 * e] = bf_lo(wlo[e]);
    xl[2 * e + 1] = bf_hi(wlo[e]);
    xh[2 * e] = bf_lo(whi[e]);
    xh[2 * e + 1] = bf_hi(whi[e]);
  }
  if (has_bias) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xl[2 * e] += bf_lo(blo[e]);
      xl[2 * e + 1] += bf_hi(blo[e]);
      xh[2 * e] += bf_lo(bhi[e]);
      xh[2 * e + 1] += bf_hi(bhi[e]);
    }
  }
}

// v: the pair narrowed to bf16.
__device__ __forceinline__ void rope_narrow(const float (&xl)[8], const float (&xh)[8], u32x4 &olo, u32x4 &ohi) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    olo[e] = f2bf_rne(xl[2 * e]) | (f2bf_rne(xl[2 * e + 1]) << 16);
    ohi[e] = f2bf_rne(xh[2 * e]) | (f2bf_rne(xh[2 * e + 1]) << 16);
  }
}

// q / k before narrowing: the pair rotated with the cos / sin chunks of the position's table row.
__device__ __forceinline__ void rope_rotate_f(const float (&xl)[8], const float (&xh)[8], u32x4 clo, u32x4 chi,
                                              u32x4 slo, u32x4 shi, float (&ol)[8], float (&oh)[8]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < 4; ++e) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int j = 2 * e + k;
      const float cl = k ? bf_hi(clo[e]) : bf_lo(clo[e]), ch = k ? bf_hi(chi[e]) : bf_lo(chi[e]);
      const float sn_l = k ? bf_hi(slo[e]) : bf_lo(slo[e]), sn_h = k ? bf_hi(shi[e]) : bf_lo(shi[e]);
      // low half: partner x[d + HD/2] with sign -1; high half: partner x[d - HD/2] with sign +1.
      ol[j] = xl[j] * cl + (-xh[j]) * sn_l;
      oh[j] = xh[j] * ch + xl[j] * sn_h;
    }
  }
}

// q / k: rotated and narrowed to bf16.
__device__ __forceinline__ void rope_rotate(const float (&xl)[8], const float (&xh)[8], u32x4 clo, u32x4 chi,
                                            u32x4 slo, u32x4 shi, u32x4 &olo, u32x4 &ohi) {
  float ol[8], oh[8];
  rope_rotate_f(xl, xh, clo, chi, slo, shi, ol, oh);
  rope_narrow(ol, oh, olo, ohi);
}

}  // namespace a8
