// The streaming vocoder's channels-last convolutions (a8_conv_cl, a8_snake_cat): the widening beside the
// attention path into the codec decoder's default conv path (serve/fast_engine.py:218-233, _CLConv.__call__:
// snake_cat then conv_cl, or conv_cl with the snake applied on its loads).
//
// Semantics follow serve/fast_kernels.py:551-615 (_conv_cl_kernel / conv_cl) and 695-729 (_snake_cat_kernel /
// snake_cat), fp16 storage:
//   conv_cl:   rows r = (b, t), t < TR; output row t*PH + p (phase p):
//              Y[b, t*PH+p, n] = bias[n] + sum_j sum_k X[b, t + j*DIL, k] W[p, j, k, n]  (+ RES[b, t*PH+p, n]),
//              X optionally passed through the snake x + ib sin(a x)^2 (fp32, rounded to fp16) on the load.
//              Products in fp16, accumulation in fp32 throughout (the reference's default F16ACC sums each
//              32-wide k slice in fp16 first; this is the more exact of the two).
//   snake_cat: Y[b] = concat(ST[b] (CTX rows), snake(X[b]) (T rows)) along time; no snake when a is null.
//
// MI355X design (an implicit GEMM: M = B*TR rows, N = Cout, K = TAPS*Cin): a workgroup computes a 64 x 64
// output tile of one phase with 4 waves (16 rows each) on v_mfma_f32_16x16x32_f16, as Y^T = W^T . X^T:
//   * X rows are the B operand straight from global memory (lane l: 16 contiguous bytes of row l % 16 at
//     channel offset 8 (l / 16)), with the snake applied in registers;
//   * each 32 x 64 weight slice [k][n] is staged once in LDS (one 16-byte load per thread) and read as the
//     A operand with ds_read_b64_tr_b16 (the LDS unit transposes 4 x 16 blocks), so W^T needs no copy;
//   * the next slice's loads are issued before the current slice's MFMAs; two barriers a slice.
// snake_cat: one lane per 8 channels of one output row, 16-byte loads and stores.
#include "a8_common.h"

namespace a8 {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mfma16x16x32_f16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                 0);
}
// fp16 word <-> fp32 (exact), two fp32 -> one dword of two fp16 (round to nearest even)
__device__ __forceinline__ float h_lo(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w)[0]; }
__device__ __forceinline__ float h_hi(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w)[1]; }
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, f16x2{(_Float16)lo, (_Float16)hi});
}
// the snake x + ib sin(a x)^2 on 8 channels (fp32, one rounding to fp16)
__device__ __forceinline__ u32x4 snake8(u32x4 v, const float *a, const float *ib) {
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float x0 = h_lo(v[j]), x1 = h_hi(v[j]);
    const float s0 = sinf(x0 * a[2 * j]), s1 = sinf(x1 * a[2 * j + 1]);
    o[j] = pack_f16x2(x0 + ib[2 * j] * s0 * s0, x1 + ib[2 * j + 1] * s1 * s1);
  }
  return o;
}

template <bool SNAKE>
__global__ __launch_bounds__(256) void k_conv_cl(const uint16_t *__restrict__ x, int64_t s_xb, int64_t s_xt,
                                                 const uint16_t *__restrict__ w, int64_t s_wp, int64_t s_wt,
                                                 int64_t s_wc, const uint16_t *__restrict__ bias,
                                                 const uint16_t *__restrict__ res, int64_t s_rb, int64_t s_rt,
                                                 uint16_t *__restrict__ y, int64_t s_yb, int64_t s_yt,
                                                 const float *__restrict__ sa, const float *__restrict__ sib, int M,
                                                 int TR, int Cin, int Cout, int CoutW, int taps, int dil, int PH) {
  warm_kernargs<160>();  // the explicit arguments above span 0x00-0x9f
  __shared__ __attribute__((aligned(16))) uint16_t wl[32 * 64];  // weight slice [k][n], 128 bytes a k row
  const int p = blockIdx.z, m0 = blockIdx.x * 64, n0 = blockIdx.y * 64;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  // this lane's X row (the B operand's column r16) and channel chunk 8g
  const int m = m0 + 16 * wv + r16;
  const bool mvalid = m < M;
  const int b = mvalid ? m / TR : 0, t = mvalid ? m - b * TR : 0;
  const uint16_t *xrow = x + (int64_t)b * s_xb + (int64_t)t * s_xt + 8 * g;
  // this thread's share of a weight slice: k row tid / 8, columns 8 (tid % 8) ..
  const int wk = tid >> 3, wn = 8 * (tid & 7);
  const uint16_t *wbase = w + (int64_t)p * s_wp + (int64_t)wk * s_wc + n0 + wn;
  const bool wcol = n0 + wn < CoutW;
  const int kchunks = (Cin + 31) / 32, steps = taps * kchunks;

  auto load_w = [&](int s) __attribute__((always_inline)) -> u32x4 {
    const int j = s / kchunks, k0 = (s - j * kchunks) * 32;
    return (wcol && k0 + wk < Cin) ? ld16(wbase + (int64_t)j * s_wt + (int64_t)k0 * s_wc) : u32x4{0u, 0u, 0u, 0u};
  };
  auto load_x = [&](int s) __attribute__((always_inline)) -> u32x4 {
    const int j = s / kchunks, k0 = (s - j * kchunks) * 32;
    if (!mvalid || k0 + 8 * g >= Cin) return u32x4{0u, 0u, 0u, 0u};
    const u32x4 v = ld16(xrow + (int64_t)j * dil * s_xt + k0);
    if (!SNAKE) return v;
    float a[8], ib[8];
    const f32x4 a0 = *reinterpret_cast<const f32x4 *>(sa + k0 + 8 * g), a1 = *reinterpret_cast<const f32x4 *>(sa + k0 + 8 * g + 4);
    const f32x4 i0 = *reinterpret_cast<const f32x4 *>(sib + k0 + 8 * g), i1 = *reinterpret_cast<const f32x4 *>(sib + k0 + 8 * g + 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      a[q] = a0[q];
      a[4 + q] = a1[q];
      ib[q] = i0[q];
      ib[4 + q] = i1[q];
    }
    return snake8(v, a, ib);
  };

  f32x4 acc[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  // A-operand reads: rows (k) 8g + r16/4 (+4), columns (n) 16 nt + 4 (r16 % 4)
  const uint16_t *ard = wl + (8 * g + (r16 >> 2)) * 64 + 4 * (r16 & 3);
  u32x4 wcur = load_w(0), xcur = load_x(0);
  for (int s = 0; s < steps; ++s) {
    st16(wl + wk * 64 + wn, wcur);
    __syncthreads();
    u32x4 wnext{0u, 0u, 0u, 0u}, xnext{0u, 0u, 0u, 0u};
    if (s + 1 < steps) {
      wnext = load_w(s + 1);
      xnext = load_x(s + 1);
    }
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const u32x2 lo = lds_tr16(ard + 16 * nt), hi = lds_tr16(ard + 16 * nt + 4 * 64);
      acc[nt] = mfma16x16x32_f16(u32x4{lo[0], lo[1], hi[0], hi[1]}, xcur, acc[nt]);
    }
    __syncthreads();
    wcur = wnext;
    xcur = xnext;
  }
  // acc[nt]: lane (r16, g) holds Y[row m][n = n0 + 16 nt + 4g + i], i = 0..3
  if (!mvalid) return;
  const int64_t orow = (int64_t)t * PH + p;
  uint16_t *yrow = y + (int64_t)b * s_yb + orow * s_yt;
  const uint16_t *rrow = res ? res + (int64_t)b * s_rb + orow * s_rt : nullptr;
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int n = n0 + 16 * nt + 4 * g;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = acc[nt][i];
      if (n + i < Cout) {
        if (bias) v[i] += h_lo(bias[n + i]);
        if (rrow) v[i] += h_lo(rrow[n + i]);
      }
    }
    if (n + 3 < Cout && (Cout & 3) == 0) {
      st8(yrow + n, u32x2{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])});
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n + i < Cout) yrow[n + i] = (uint16_t)(pack_f16x2(v[i], 0.f) & 0xffffu);
    }
  }
}

template <bool SNAKE>
__global__ __launch_bounds__(256) void k_snake_cat(const uint16_t *__restrict__ x, int64_t s_xb, int64_t s_xt,
                                                   const uint16_t *__restrict__ st, int64_t s_sb, int64_t s_st,
                                                   const float *__restrict__ sa, const float *__restrict__ sib,
                                                   uint16_t *__restrict__ y, int64_t s_yb, int64_t s_yt, int B,
                                                   int T, int CTX, int C) {
  warm_kernargs<104>();  // the explicit arguments above span 0x00-0x67
  const int nch = C >> 3, rows = CTX + T;
  const uint32_t id = blockIdx.x * 256u + threadIdx.x;
  if (id >= (uint32_t)B * (uint32_t)rows * (uint32_t)nch) return;
  const int c = (int)(id % (uint32_t)nch);
  const uint32_t rt = id / (uint32_t)nch;
  const int tt = (int)(rt % (uint32_t)rows), b = (int)(rt / (uint32_t)rows);
  u32x4 v;
  if (tt < CTX) {
    v = ld16(st + (int64_t)b * s_sb + (int64_t)tt * s_st + 8 * c);
  } else {
    v = ld16(x + (int64_t)b * s_xb + (int64_t)(tt - CTX) * s_xt + 8 * c);
    if (SNAKE) {
      float a[8], ib[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        a[q] = sa[8 * c + q];
        ib[q] = sib[8 * c + q];
      }
      v = snake8(v, a, ib);
    }
  }
  st16(y + (int64_t)b * s_yb + (int64_t)tt * s_yt + 8 * c, v);
}

static inline bool al16(const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

}  // namespace a8

extern "C" int a8_conv_cl(const void *x, int64_t s_xb, int64_t s_xt, const void *w, int64_t s_wp, int64_t s_wt,
                          int64_t s_wc, int cout_w, const void *bias, const void *res, int64_t s_rb, int64_t s_rt,
                          void *y, int64_t s_yb, int64_t s_yt, const float *snake_a, const float *snake_ib, int B,
                          int Tin, int TR, int Cin, int Cout, int taps, int dil, int ph, void *stream) {
  using namespace a8;
  if (B < 0 || TR < 0 || Cin <= 0 || Cout <= 0 || taps <= 0 || dil <= 0 || ph <= 0 || cout_w < Cout)
    return set_error(A8_EINVAL, "conv_cl: bad sizes B=%d TR=%d Cin=%d Cout=%d taps=%d dil=%d ph=%d cout_w=%d", B, TR,
                     Cin, Cout, taps, dil, ph, cout_w);
  if ((int64_t)TR + (int64_t)(taps - 1) * dil > Tin)
    return set_error(A8_EINVAL, "conv_cl: %d input rows, %d needed", Tin, TR + (taps - 1) * dil);
  if (Cin % 8) return set_error(A8_EUNSUP, "conv_cl: Cin %d not a multiple of 8", Cin);
  if (B == 0 || TR == 0) return 0;
  if (!x || !w || !y || (snake_a != nullptr) != (snake_ib != nullptr))
    return set_error(A8_EINVAL, "conv_cl: null pointer");
  if (!al16(x) || !al16(w) || (s_xb | s_xt | s_wp | s_wt | s_wc) & 7 || (cout_w & 7) ||
      (snake_a && (!al16(snake_a) || !al16(snake_ib))) || (reinterpret_cast<uintptr_t>(y) & 7u) ||
      ((Cout & 3) == 0 && (s_yb | s_yt) & 3))
    return set_error(A8_EALIGN, "conv_cl: x / w / snake 16-byte aligned, strides multiples of 8, y 8-byte");
  const int64_t M = (int64_t)B * TR;
  if (M > INT32_MAX / 2) return set_error(A8_EUNSUP, "conv_cl: %lld rows too many", (long long)M);
  const dim3 grid((unsigned)((M + 63) / 64), (unsigned)((Cout + 63) / 64), (unsigned)ph);
#define A8_CONV_ARGS (const uint16_t *)x, s_xb, s_xt, (const uint16_t *)w, s_wp, s_wt, s_wc, (const uint16_t *)bias, \
                     (const uint16_t *)res, s_rb, s_rt, (uint16_t *)y, s_yb, s_yt, snake_a, snake_ib, (int)M, TR, Cin, \
                     Cout, cout_w, taps, dil, ph
  if (snake_a)
    hipLaunchKernelGGL(k_conv_cl<true>, grid, dim3(256), 0, (hipStream_t)stream, A8_CONV_ARGS);
  else
    hipLaunchKernelGGL(k_conv_cl<false>, grid, dim3(256), 0, (hipStream_t)stream, A8_CONV_ARGS);
#undef A8_CONV_ARGS
  return (int)hipGetLastError();
}

extern "C" int a8_snake_cat(const void *x, int64_t s_xb, int64_t s_xt, const void *state, int64_t s_sb, int64_t s_st,
                            const float *a, const float *ib, void *y, int64_t s_yb, int64_t s_yt, int B, int T, int CTX,
                            int C, void *stream) {
  using namespace a8;
  if (B < 0 || T < 0 || CTX < 0 || C <= 0) return set_error(A8_EINVAL, "snake_cat: bad sizes B=%d T=%d CTX=%d C=%d", B, T, CTX, C);
  if (C % 8) return set_error(A8_EUNSUP, "snake_cat: C %d not a multiple of 8", C);
  if (B == 0 || T + CTX == 0) return 0;
  if ((T > 0 && !x) || (CTX > 0 && !state) || !y || (a != nullptr) != (ib != nullptr))
    return set_error(A8_EINVAL, "snake_cat: null pointer");
  if ((x && !al16(x)) || (state && !al16(state)) || !al16(y) || (a && (!al16(a) || !al16(ib))) ||
      (s_xb | s_xt | s_sb | s_st | s_yb | s_yt) & 7)
    return set_error(A8_EALIGN, "snake_cat: pointers 16-byte aligned, strides multiples of 8");
  const int64_t n = (int64_t)B * (CTX + T) * (C / 8);
  if (n >= (int64_t)1 << 31) return set_error(A8_EUNSUP, "snake_cat: too large");
  const unsigned grid = (unsigned)((n + 255) / 256);
  if (a)
    hipLaunchKernelGGL(k_snake_cat<true>, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const uint16_t *)x, s_xb, s_xt,
                       (const uint16_t *)state, s_sb, s_st, a, ib, (uint16_t *)y, s_yb, s_yt, B, T, CTX, C);
  else
    hipLaunchKernelGGL(k_snake_cat<false>, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const uint16_t *)x, s_xb,
                       s_xt, (const uint16_t *)state, s_sb, s_st, a, ib, (uint16_t *)y, s_yb, s_yt, B, T, CTX, C);
  return (int)hipGetLastError();
}
