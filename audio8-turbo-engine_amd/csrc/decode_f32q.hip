// Decode attention with fp32 queries (a8_decode_attn_f32q): the reference's PREC = "ieee" branch of the
// split kernel (serve/fast_kernels.py:193-235, chosen at 279 when q is float32) and its combine (238-253).
//
// Semantics: for each row and q head, s = (q . k) * scale with q in fp32 and k bf16 widened exactly, fp32
// products and sums (ieee: no input rounding); online softmax in natural-exp units; the weights rounded to
// bf16 (p.to(v.dtype)) for P.V with fp32 accumulation, the row sum l of the unrounded fp32 weights; the key
// ranges of the workgroup's four waves merged as the combine merges splits, out = num / den, stored as
// bf16 or fp32 (the output tensor's dtype). lens 0 gives 0 / 0 = NaN, as the reference; lens past the cache
// attend the whole cache row.
//
// The engine never decodes an fp32 query (its q rows are bf16), so this is a plain, exact VALU kernel, not a
// tuned one: a workgroup per (row, kv head), four waves taking 64-key tiles in turn. Per tile a lane holds
// one key for the scores (its K row straight from memory, q broadcast from LDS), the weights and the V tile
// go through the wave's own LDS area, and for P.V a lane holds one (or two) head dims.
#include "a8_common.h"

namespace a8 {
namespace {

constexpr int kFqWaves = 4;
constexpr int kFqMaxG = 16;    // q heads per kv head
constexpr int kFqMaxHD = 128;

template <int HD>
__global__ __launch_bounds__(64 * kFqWaves, 1) void k_decode_f32q(
    const float *__restrict__ q, int64_t s_qb, int64_t s_qh, const uint16_t *__restrict__ kc,
    const uint16_t *__restrict__ vc, int64_t s_kb, int64_t s_kh, int64_t s_ks, int cache_rows, int cache_len,
    const int32_t *__restrict__ lens, const int32_t *__restrict__ rowmap, void *__restrict__ out, int64_t s_ob,
    int64_t s_oh, int out_f32, int nkv, int group, float scale) {
  static_assert(HD % 64 == 0 && HD <= kFqMaxHD, "head dims");
  constexpr int DPL = HD / 64;  // head dims per lane in P.V
  __shared__ float qs[kFqMaxG * HD];
  __shared__ float ps[kFqWaves][kFqMaxG][64];
  __shared__ __attribute__((aligned(16))) uint16_t vs[kFqWaves][64 * HD];
  __shared__ float mrg_m[kFqWaves][kFqMaxG], mrg_l[kFqWaves][kFqMaxG];
  __shared__ float mrg_a[kFqWaves][kFqMaxG * HD];

  const int row = blockIdx.x / nkv, kh = blockIdx.x - row * nkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int crow = rowmap ? rowmap[row] : row;
  const bool ok = crow >= 0 && crow < cache_rows;
  const int L = ok ? min(max(lens[row], 0), cache_len) : 0;

  for (int i = tid; i < group * HD; i += 64 * kFqWaves) {
    const int h = i / HD, d = i - h * HD;
    qs[i] = q[(int64_t)row * s_qb + (int64_t)(kh * group + h) * s_qh + d];
  }
  __syncthreads();

  const uint16_t *kb = kc + (int64_t)(ok ? crow : 0) * s_kb + (int64_t)kh * s_kh;
  const uint16_t *vb = vc + (int64_t)(ok ? crow : 0) * s_kb + (int64_t)kh * s_kh;
  float m[kFqMaxG], l[kFqMaxG], acc[kFqMaxG][DPL];
#pragma unroll
  for (int h = 0; h < kFqMaxG; ++h) {
    m[h] = -__builtin_inff();
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[h][e] = 0.f;
  }
  const int ntile = (L + 63) / 64;
  for (int t = w; t < ntile; t += kFqWaves) {
    const int n = 64 * t + lane;
    const bool valid = n < L;
    // this lane's key: its scores for every q head (fp32 products, the key widened exactly)
    float s[kFqMaxG];
#pragma unroll
    for (int h = 0; h < kFqMaxG; ++h) s[h] = 0.f;
    u32x4 vrow[HD / 8];
#pragma unroll
    for (int c = 0; c < HD / 8; ++c) {
      const u32x4 kv = valid ? ld16(kb + (int64_t)n * s_ks + 8 * c) : u32x4{0u, 0u, 0u, 0u};
      vrow[c] = valid ? ld16(vb + (int64_t)n * s_ks + 8 * c) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float kf = (j & 1) ? bf_hi(kv[j >> 1]) : bf_lo(kv[j >> 1]);
#pragma unroll
        for (int h = 0; h < kFqMaxG; ++h)
          if (h < group) s[h] = __builtin_fmaf(qs[h * HD + 8 * c + j], kf, s[h]);
      }
    }
    // the V tile into this wave's LDS area (rows past L are zeros: masked loads read 0.0)
#pragma unroll
    for (int c = 0; c < HD / 8; ++c) st16(&vs[w][lane * HD + 8 * c], vrow[c]);
    // online softmax per head over the tile's 64 keys (one per lane)
#pragma unroll
    for (int h = 0; h < kFqMaxG; ++h) {
      if (h >= group) continue;
      const float sv = valid ? s[h] * scale : -__builtin_inff();
      float tm = sv;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) tm = fmaxf(tm, __shfl_xor(tm, o));
      const float mn = fmaxf(m[h], tm);  // finite: a tile holds at least one key below L
      const float alpha = expf(m[h] - mn);
      const float p = expf(sv - mn);
      float ts = p;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) ts += __shfl_xor(ts, o);
      l[h] = l[h] * alpha + ts;
      m[h] = mn;
      ps[w][h][lane] = bf_lo(pack_bf16x2(p, 0.f));  // p.to(v.dtype)
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[h][e] *= alpha;
    }
    // the wave's own LDS writes are done (lgkmcnt(0)) before any lane reads another lane's; the wave runs in
    // lockstep, so no workgroup barrier is needed (and the waves take different tile counts)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
    // P.V: lane = head dim(s)
#pragma unroll 4
    for (int j = 0; j < 64; ++j) {
      float vv[DPL];
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        const uint16_t hv = vs[w][j * HD + lane + 64 * e];
        vv[e] = __uint_as_float((uint32_t)hv << 16);
      }
#pragma unroll
      for (int h = 0; h < kFqMaxG; ++h) {
        if (h >= group) continue;
        const float pj = ps[w][h][j];
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[h][e] = __builtin_fmaf(pj, vv[e], acc[h][e]);
      }
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();  // the next tile rewrites ps / vs
    asm volatile("" ::: "memory");
  }
  // merge the waves' key ranges as the combine merges splits
#pragma unroll
  for (int h = 0; h < kFqMaxG; ++h) {
    if (h >= group) continue;
    if (lane == 0) {
      mrg_m[w][h] = m[h];
      mrg_l[w][h] = l[h];
    }
#pragma unroll
    for (int e = 0; e < DPL; ++e) mrg_a[w][h * HD + lane + 64 * e] = acc[h][e];
  }
  __syncthreads();
  for (int i = tid; i < group * HD; i += 64 * kFqWaves) {
    const int h = i / HD, d = i - h * HD;
    float M = -__builtin_inff();
#pragma unroll
    for (int v = 0; v < kFqWaves; ++v) M = fmaxf(M, mrg_m[v][h]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int v = 0; v < kFqWaves; ++v) {
      const float wt = mrg_m[v][h] == -__builtin_inff() ? 0.f : expf(mrg_m[v][h] - M);
      num += mrg_a[v][i] * wt;
      den += mrg_l[v][h] * wt;
    }
    const float o = num / den;
    const int64_t oo = (int64_t)row * s_ob + (int64_t)(kh * group + h) * s_oh + d;
    if (out_f32)
      reinterpret_cast<float *>(out)[oo] = o;
    else
      reinterpret_cast<uint16_t *>(out)[oo] = (uint16_t)(pack_bf16x2(o, 0.f) & 0xffffu);
  }
}

}  // namespace
}  // namespace a8

extern "C" int a8_decode_attn_f32q(const float *q, int64_t s_qb, int64_t s_qh, const void *kc, const void *vc,
                                   int64_t s_kb, int64_t s_kh, int64_t s_ks, int cache_rows, int cache_len,
                                   const int32_t *lens, const int32_t *rowmap, void *out, int64_t s_ob, int64_t s_oh,
                                   int out_f32, int b, int nq, int nkv, int hd, float scale, void *stream) {
  using namespace a8;
  if (b < 0 || nq <= 0 || nkv <= 0 || nq % nkv || cache_rows < 0 || cache_len < 0)
    return set_error(A8_EINVAL, "decode_attn_f32q: bad sizes b=%d nq=%d nkv=%d", b, nq, nkv);
  if (hd != 64 && hd != 128) return set_error(A8_EUNSUP, "decode_attn_f32q: head_dim %d (64 or 128)", hd);
  const int group = nq / nkv;
  if (group > kFqMaxG) return set_error(A8_EUNSUP, "decode_attn_f32q: %d q heads per kv head (at most %d)", group,
                                        kFqMaxG);
  if (b == 0) return 0;
  if (!q || !kc || !vc || !lens || !out) return set_error(A8_EINVAL, "decode_attn_f32q: null pointer");
  if ((reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc)) & 15u || (s_kb | s_kh | s_ks) & 7 ||
      s_ks < hd)
    return set_error(A8_EALIGN, "decode_attn_f32q: caches 16-byte aligned, strides multiples of 8, rows >= hd");
  const dim3 grid((unsigned)((int64_t)b * nkv));
  if (hd == 64)
    hipLaunchKernelGGL(k_decode_f32q<64>, grid, dim3(64 * kFqWaves), 0, (hipStream_t)stream, q, s_qb, s_qh,
                       (const uint16_t *)kc, (const uint16_t *)vc, s_kb, s_kh, s_ks, cache_rows, cache_len, lens,
                       rowmap, out, s_ob, s_oh, out_f32, nkv, group, scale);
  else
    hipLaunchKernelGGL(k_decode_f32q<128>, grid, dim3(64 * kFqWaves), 0, (hipStream_t)stream, q, s_qb, s_qh,
                       (const uint16_t *)kc, (const uint16_t *)vc, s_kb, s_kh, s_ks, cache_rows, cache_len, lens,
                       rowmap, out, s_ob, s_oh, out_f32, nkv, group, scale);
  return (int)hipGetLastError();
}
