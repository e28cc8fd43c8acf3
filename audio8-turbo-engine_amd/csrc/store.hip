// Fused qkv bias + rotate_half RoPE + K/V store (a8_bias_rope_store).
//
// Semantics follow serve/fast_kernels.py:139-187 (_bias_rope_store_kernel / bias_rope_store), for a head
// dimension HD (a multiple of 16, <= 256; the reference's HD constexpr): per token row r and head h of the
// fused [q | k | v] row,
//   x  = f32(qkv[r, h*HD + d]) + f32(bias[h*HD + d])
//   q/k: o[d] = bf16(x[d]*cos[pos, d] + sign(d) * x[(d+HD/2) % HD] * sin[pos, d]),  sign = -1 for d < HD/2
//   v:   o[d] = bf16(x[d])
// q goes to qo[r, h]; k / v go to kc / vc[slot[r], h', pos[r] % ring]. qo may be null: then only the k / v heads
// are launched (the fused prefill, a8_prefill_attn_qkv, forms q itself from the same qkv rows).
//
// MI355X layout: one thread owns the partner pair of 16-byte chunks (d = 8c..8c+7 and HD/2+8c..)
// of one head, so rotate_half needs no cross-lane traffic and every global access is a 128-bit
// load/store; HD/16 consecutive lanes cover one head row (4 for the engine's HD = 64). The work is ~1 MB
// per layer at 192 slots: the kernel is launch-latency bound and sized as a single flat grid.
#include "rope.h"

namespace a8 {

__global__ __launch_bounds__(256) void k_bias_rope_store(
    const uint16_t *__restrict__ qkv, int64_t s_qkv, const uint16_t *__restrict__ bias,
    const uint16_t *__restrict__ cos_tab, const uint16_t *__restrict__ sin_tab, int64_t s_cs, int n_tab,
    const int32_t *__restrict__ pos, const int32_t *__restrict__ slot, int R,
    uint16_t *__restrict__ qo, int64_t s_qo_r, int64_t s_qo_h,
    uint16_t *__restrict__ kc, uint16_t *__restrict__ vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
    int cache_rows, int cache_len, int nq, int nkv, int ring, int hd) {
  warm_kernargs<168>();  // the explicit arguments above span 0x00-0xa7
  const int h0 = qo ? 0 : nq;              // first head launched: the k heads when q is not wanted
  const int H = nq + 2 * nkv - h0;
  const int np = hd >> 4;                  // chunk pairs (threads) per head
  const int half = hd >> 1;                // the partner chunk's offset
  const uint32_t per = (uint32_t)np * (uint32_t)H;  // threads per row (the host keeps R * per below 2^31)
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  if (t >= (uint32_t)R * per) return;
  const int r = (int)(t / per);
  const int rem = (int)(t - (uint32_t)r * per);
  const int h = h0 + rem / np, c = rem - (h - h0) * np;

  // Every load that does not depend on the position goes out before anything waits for it; the position
  // check only decides the stores (so the loads are not held behind it).
  const int p = pos[r];
  const int64_t sl = slot[r];
  const uint16_t *src = qkv + (int64_t)r * s_qkv + h * hd;
  const u32x4 wlo = ld16(src + 8 * c), whi = ld16(src + half + 8 * c);
  u32x4 blo{0u, 0u, 0u, 0u}, bhi{0u, 0u, 0u, 0u};
  if (bias) {
    blo = ld16(bias + h * hd + 8 * c);
    bhi = ld16(bias + h * hd + half + 8 * c);
  }
  const bool in_tab = p >= 0 && p < n_tab;  // a position outside the RoPE tables: the row writes nothing
  const int sidx = p % ring;
  const bool store_ok = in_tab && sl >= 0 && sl < cache_rows && sidx < cache_len;
  float xl[8], xh[8];
  rope_x(wlo, whi, blo, bhi, bias != nullptr, xl, xh);

  u32x4 olo, ohi;
  if (h >= nq + nkv) {  // v head: bias only
    if (!store_ok) return;
    rope_narrow(xl, xh, olo, ohi);
    uint16_t *dst = vc + sl * s_kb + (int64_t)(h - nq - nkv) * s_kh + (int64_t)sidx * s_ks;
    st16(dst + 8 * c, olo);
    st16(dst + half + 8 * c, ohi);
    return;
  }

  const int pc = in_tab ? p : 0;  // the host launches nothing when the tables are empty
  const uint16_t *crow = cos_tab + (int64_t)pc * s_cs, *srow = sin_tab + (int64_t)pc * s_cs;
  rope_rotate(xl, xh, ld16(crow + 8 * c), ld16(crow + half + 8 * c), ld16(srow + 8 * c), ld16(srow + half + 8 * c),
              olo, ohi);
  if (!in_tab) return;
  uint16_t *dst;
  if (h < nq) {
    dst = qo + (int64_t)r * s_qo_r + (int64_t)h * s_qo_h;
  } else {
    if (!store_ok) return;
    dst = kc + sl * s_kb + (int64_t)(h - nq) * s_kh + (int64_t)sidx * s_ks;
  }
  st16(dst + 8 * c, olo);
  st16(dst + half + 8 * c, ohi);
}

static inline bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace a8

extern "C" int a8_bias_rope_store(const void *qkv, int64_t s_qkv, const void *bias,
                                  const void *cos_tab, const void *sin_tab, int64_t s_cs, int n_tab,
                                  const int32_t *pos, const int32_t *slot, int R,
                                  void *qo, int64_t s_qo_r, int64_t s_qo_h,
                                  void *kc, void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                                  int cache_rows, int cache_len,
                                  int nq, int nkv, int hd, int ring, void *stream) {
  using namespace a8;
  if (hd <= 0 || hd > 256 || hd % 16)
    return set_error(A8_EUNSUP, "bias_rope_store: head_dim %d not supported (a multiple of 16 up to 256)", hd);
  if (R < 0 || nq <= 0 || nkv <= 0 || ring <= 0 || n_tab < 0 || cache_rows < 0 || cache_len < 0)
    return set_error(A8_EINVAL, "bias_rope_store: bad sizes R=%d nq=%d nkv=%d ring=%d n_tab=%d", R, nq, nkv,
                     ring, n_tab);
  if (R == 0) return 0;
  if (!qkv || !cos_tab || !sin_tab || !pos || !slot || !kc || !vc)
    return set_error(A8_EINVAL, "bias_rope_store: null pointer");
  if (!al16(qkv) || !al16(cos_tab) || !al16(sin_tab) || (qo && !al16(qo)) || !al16(kc) || !al16(vc) ||
      (bias && !al16(bias)) || (s_qkv | s_cs | s_qo_r | s_qo_h | s_kb | s_kh | s_ks) & 7)
    return set_error(A8_EALIGN, "bias_rope_store: pointers must be 16-byte aligned and strides multiples of 8");
  const int64_t threads = (int64_t)R * ((qo ? nq : 0) + 2 * nkv) * (hd / 16);
  if (threads >= (int64_t)1 << 31) return set_error(A8_EUNSUP, "bias_rope_store: %d rows x %d heads too many", R, nq + 2 * nkv);
  if (n_tab == 0) return 0;  // no position is inside the tables: nothing is written
  const unsigned grid = (unsigned)((threads + 255) / 256);
  hipLaunchKernelGGL(k_bias_rope_store, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t *)qkv, s_qkv, (const uint16_t *)bias, (const uint16_t *)cos_tab,
                     (const uint16_t *)sin_tab, s_cs, n_tab, pos, slot, R, (uint16_t *)qo, s_qo_r, s_qo_h,
                     (uint16_t *)kc, (uint16_t *)vc, s_kb, s_kh, s_ks, cache_rows, cache_len, nq, nkv, ring, hd);
  return (int)hipGetLastError();
}
