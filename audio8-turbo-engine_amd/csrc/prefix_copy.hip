// A voice prefix's K/V into the cache rows of the requests that use it (a8_prefix_copy).
//
// Semantics follow serve/fast_engine.py:1098-1103 (FastEngine._prefill, step 1): the prefix K and V of one
// voice, [layers, nkv, Lp, hd] each (computed once by _prefix_kv, 1073-1087), go to every slot s of the
// group: kc_all[l, s, h, p, :] = k[l, h, p, :] and vc_all[...] = v[...] for p < Lp -- the reference's two
// torch index-puts `kc_all[:, idx, :, :Lp] = k.unsqueeze(1)` / `vc_all[...] = v.unsqueeze(1)` in one launch.
//
// MI355X design (HBM-write bound: the prefix is read from L2 / MALL once per slot, the slots' rows are
// written once): for each (K or V, layer, slot, kv head) the Lp positions are one contiguous run of
// Lp * hd * 2 bytes on both sides (positions are contiguous rows of a head), so a workgroup copies an 8 KB
// piece of one run -- 256 lanes x two 16-byte loads in flight, then the two stores, non-temporal (the
// rows are not read again by this launch) -- and the grid is pieces x runs, tens of thousands of
// workgroups for the engine's admission (64 slots x 24 layers x 2 heads). Measured at that size (4 voices
// x 16 slots, 250 MB): 51.9 us = 4.8 TB/s; four loads per lane 59.7 us, plain stores 58.6 us.
#include "a8_common.h"

namespace a8 {

constexpr int kPcLanes = 256;
constexpr int kPcUnroll = 2;
constexpr int kPcPiece = kPcLanes * kPcUnroll * 16;  // bytes of a run one workgroup copies

__global__ __launch_bounds__(kPcLanes) void k_prefix_copy(
    const uint16_t *__restrict__ sk, const uint16_t *__restrict__ sv, int64_t s_l, int64_t s_h,
    uint16_t *__restrict__ dk, uint16_t *__restrict__ dv, int64_t d_l, int64_t d_r, int64_t d_h,
    const int32_t *__restrict__ slots, int n, int layers, int nkv, uint32_t bytes, int cache_rows, int pieces) {
  warm_kernargs<104>();  // the explicit arguments above span 0x00-0x67
  // blockIdx.x = piece + pieces * run; run = ((kv * layers + l) * n + i) * nkv + h
  const int piece = blockIdx.x % pieces;
  int run = blockIdx.x / pieces;
  const int h = run % nkv;
  run /= nkv;
  const int i = run % n;
  run /= n;
  const int l = run % layers;
  const bool is_v = run >= layers;
  const int64_t s = slots[i];
  if (s < 0 || s >= cache_rows) return;  // a slot outside the cache: nothing is written
  const char *src = reinterpret_cast<const char *>((is_v ? sv : sk) + (int64_t)l * s_l + (int64_t)h * s_h);
  char *dst = reinterpret_cast<char *>((is_v ? dv : dk) + (int64_t)l * d_l + s * d_r + (int64_t)h * d_h);
  const uint32_t base = (uint32_t)piece * kPcPiece + threadIdx.x * 16u;
  u32x4 v[kPcUnroll] = {};
#pragma unroll
  for (int u = 0; u < kPcUnroll; ++u) {
    const uint32_t o = base + u * kPcLanes * 16u;
    if (o < bytes) v[u] = ld16(src + o);
  }
#pragma unroll
  for (int u = 0; u < kPcUnroll; ++u) {
    const uint32_t o = base + u * kPcLanes * 16u;
    if (o < bytes) __builtin_nontemporal_store(v[u], reinterpret_cast<u32x4 *>(dst + o));
  }
}

static inline bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace a8

extern "C" int a8_prefix_copy(const void *k, const void *v, int64_t s_l, int64_t s_h, int64_t s_p,
                              void *kc_all, void *vc_all, int64_t d_l, int64_t d_r, int64_t d_h, int64_t d_p,
                              const int32_t *slots, int n, int layers, int nkv, int Lp, int hd, int cache_rows,
                              int cache_len, void *stream) {
  using namespace a8;
  if (hd <= 0 || hd > 256 || hd % 8)
    return set_error(A8_EUNSUP, "prefix_copy: head_dim %d not supported (a multiple of 8 up to 256)", hd);
  if (n < 0 || layers < 0 || nkv <= 0 || Lp < 0 || cache_rows < 0 || cache_len < 0)
    return set_error(A8_EINVAL, "prefix_copy: bad sizes n=%d layers=%d nkv=%d Lp=%d", n, layers, nkv, Lp);
  if (Lp > cache_len) return set_error(A8_EINVAL, "prefix_copy: prefix of %d positions > cache length %d", Lp, cache_len);
  if (n == 0 || layers == 0 || Lp == 0) return 0;
  if (!k || !v || !kc_all || !vc_all || !slots) return set_error(A8_EINVAL, "prefix_copy: null pointer");
  if (s_p != hd || d_p != hd)  // a head's positions are contiguous rows on both sides
    return set_error(A8_EUNSUP, "prefix_copy: positions must be contiguous rows (s_p %lld, d_p %lld)",
                     (long long)s_p, (long long)d_p);
  if (!al16(k) || !al16(v) || !al16(kc_all) || !al16(vc_all) || (s_l | s_h | d_l | d_r | d_h) & 7)
    return set_error(A8_EALIGN, "prefix_copy: pointers must be 16-byte aligned and strides multiples of 8");
  const int64_t bytes = (int64_t)Lp * hd * 2;  // one run
  if (bytes >= ((int64_t)1 << 31)) return set_error(A8_EUNSUP, "prefix_copy: a run of %lld bytes too long", (long long)bytes);
  const int pieces = (int)((bytes + kPcPiece - 1) / kPcPiece);
  const int64_t grid = (int64_t)pieces * nkv * n * layers * 2;
  if (grid > INT32_MAX) return set_error(A8_EUNSUP, "prefix_copy: %lld workgroups too many", (long long)grid);
  hipLaunchKernelGGL(k_prefix_copy, dim3((unsigned)grid), dim3(kPcLanes), 0, (hipStream_t)stream,
                     (const uint16_t *)k, (const uint16_t *)v, s_l, s_h, (uint16_t *)kc_all, (uint16_t *)vc_all, d_l,
                     d_r, d_h, slots, n, layers, nkv, (uint32_t)bytes, cache_rows, pieces);
  return (int)hipGetLastError();
}
