// The slow-AR layer's element-wise steps on either side of the attention path: residual add + RMSNorm
// (a8_rmsnorm) and the gated MLP activation (a8_silu_mul).
//
// Semantics follow serve/fast_kernels.py:30-69 (_rmsnorm_kernel / rmsnorm) and 526-545 (_silu_mul_kernel /
// silu_mul):
//   rmsnorm:  with a residual, h = bf16(f32(x) + f32(r)), stored to res_out; without, h = x.
//             var = sum(f32(h)^2) / N; xn = bf16(f32(h) * rsqrt(var + eps)); y = bf16(f32(w) * f32(xn)).
//   silu_mul: g = gu[:, :I], u = gu[:, I:]; gs = bf16(g / (1 + exp(-g))); y = bf16(f32(gs) * f32(u)).
//
// MI355X design (HBM bound: 2-7 KB per row, a few MB per launch at the engine's batch): rmsnorm -- one wave
// per row, lane l owns the 16-byte chunks l, l + 64, ... (8 values each), which stay in registers between
// the sum of squares (reduced across the wave by xor shuffles) and the output; silu_mul -- one lane per 8
// outputs, 16-byte loads of g and u, 16-byte stores.
#include "a8_common.h"

namespace a8 {

constexpr int kRnMaxChunks = 4;  // 16-byte chunks per lane: rows of up to 64 x 4 x 8 = 2048 values

template <bool RES>
__global__ __launch_bounds__(256) void k_rmsnorm(const uint16_t *__restrict__ x, int64_t sx,
                                                 const uint16_t *r, int64_t sr, const uint16_t *__restrict__ w,
                                                 uint16_t *__restrict__ y, int64_t sy, uint16_t *ro, int64_t sro,
                                                 int rows, int N, float eps) {
  warm_kernargs<84>();  // the explicit arguments above span 0x00-0x53
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int nch = N >> 3;
  // every load of the row -- x, the residual and the norm weight -- goes out before the first use: one memory
  // round trip, not one for the row and another for the weight after the reduction
  // (buffer loads: chunks past the row read zeros through the range check, so no branch splits the batch)
  const rsrc_t xr = make_rsrc(x + (int64_t)row * sx, (uint32_t)N * 2u), wr = make_rsrc(w, (uint32_t)N * 2u);
  const rsrc_t rr = make_rsrc(RES ? r + (int64_t)row * sr : x, RES ? (uint32_t)N * 2u : 0u);
  u32x4 h[kRnMaxChunks], rv[kRnMaxChunks], wv[kRnMaxChunks];
#pragma unroll
  for (int c = 0; c < kRnMaxChunks; ++c) {
    const uint32_t off = (uint32_t)(lane + 64 * c) * 16u;
    h[c] = bld16(xr, off);
    rv[c] = RES ? bld16(rr, off) : u32x4{0u, 0u, 0u, 0u};
    wv[c] = bld16(wr, off);
  }
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kRnMaxChunks; ++c) {
    const int ch = lane + 64 * c;
    if (ch >= nch) continue;
    u32x4 v = h[c];
    if (RES) {  // residual add in fp32, rounded once to bf16 (the new residual stream)
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = pack_bf16x2(bf_lo(v[j]) + bf_lo(rv[c][j]), bf_hi(v[j]) + bf_hi(rv[c][j]));
      st16(ro + (int64_t)row * sro + 8 * ch, v);
      h[c] = v;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = bf_lo(v[j]), b = bf_hi(v[j]);
      ss += a * a + b * b;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
  const float inv = __builtin_amdgcn_rsqf(ss / (float)N + eps);
#pragma unroll
  for (int c = 0; c < kRnMaxChunks; ++c) {
    const int ch = lane + 64 * c;
    if (ch >= nch) continue;
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t xn = pack_bf16x2(bf_lo(h[c][j]) * inv, bf_hi(h[c][j]) * inv);  // HF: .to(input dtype)
      o[j] = pack_bf16x2(bf_lo(wv[c][j]) * bf_lo(xn), bf_hi(wv[c][j]) * bf_hi(xn));   // HF: weight * x
    }
    st16(y + (int64_t)row * sy + 8 * ch, o);
  }
}

__global__ __launch_bounds__(256) void k_silu_mul(const uint16_t *__restrict__ gu, int64_t s_gu,
                                                  uint16_t *__restrict__ y, int64_t s_y, int rows, int I) {
  warm_kernargs<40>();  // the explicit arguments above span 0x00-0x27
  const int nch = I >> 3;
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  if (t >= (uint32_t)rows * (uint32_t)nch) return;
  const int r = (int)(t / (uint32_t)nch), c = (int)(t - (uint32_t)r * (uint32_t)nch);
  const uint16_t *p = gu + (int64_t)r * s_gu + 8 * c;
  const u32x4 g = ld16(p), u = ld16(p + I);
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = silu_mul_bf16x2(g[j], u[j]);
  st16(y + (int64_t)r * s_y + 8 * c, o);
}

static inline bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace a8

extern "C" int a8_rmsnorm(const void *x, int64_t sx, const void *residual, int64_t sr, const void *w, void *y,
                          int64_t sy, void *res_out, int64_t sro, int rows, int N, float eps, void *stream) {
  using namespace a8;
  if (rows < 0 || N <= 0 || N % 8 || N > 64 * kRnMaxChunks * 8)
    return set_error(A8_EUNSUP, "rmsnorm: rows %d, width %d (a multiple of 8 up to %d)", rows, N, 64 * kRnMaxChunks * 8);
  if (rows == 0) return 0;
  if (!x || !w || !y || (residual && !res_out)) return set_error(A8_EINVAL, "rmsnorm: null pointer");
  if (!al16(x) || !al16(w) || !al16(y) || (residual && (!al16(residual) || !al16(res_out))) ||
      (sx | sy | (residual ? (sr | sro) : 0)) & 7)
    return set_error(A8_EALIGN, "rmsnorm: pointers must be 16-byte aligned and strides multiples of 8");
  const unsigned grid = (unsigned)((rows + 3) / 4);
  if (residual)
    hipLaunchKernelGGL(k_rmsnorm<true>, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const uint16_t *)x, sx,
                       (const uint16_t *)residual, sr, (const uint16_t *)w, (uint16_t *)y, sy, (uint16_t *)res_out, sro,
                       rows, N, eps);
  else
    hipLaunchKernelGGL(k_rmsnorm<false>, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const uint16_t *)x, sx,
                       (const uint16_t *)nullptr, (int64_t)0, (const uint16_t *)w, (uint16_t *)y, sy, (uint16_t *)nullptr,
                       (int64_t)0, rows, N, eps);
  return (int)hipGetLastError();
}

extern "C" int a8_silu_mul(const void *gu, int64_t s_gu, void *y, int64_t s_y, int rows, int I, void *stream) {
  using namespace a8;
  if (rows < 0 || I <= 0 || I % 8) return set_error(A8_EUNSUP, "silu_mul: rows %d, width %d (a multiple of 8)", rows, I);
  if (rows == 0) return 0;
  if (!gu || !y) return set_error(A8_EINVAL, "silu_mul: null pointer");
  if (!al16(gu) || !al16(y) || (s_gu | s_y) & 7)
    return set_error(A8_EALIGN, "silu_mul: pointers must be 16-byte aligned and strides multiples of 8");
  const int64_t threads = (int64_t)rows * (I / 8);
  if (threads >= (int64_t)1 << 31) return set_error(A8_EUNSUP, "silu_mul: %d rows x %d too many", rows, I);
  hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t *)gu, s_gu, (uint16_t *)y, s_y, rows, I);
  return (int)hipGetLastError();
}
