// Device helpers shared by the attention kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/a8attn.h"

namespace a8 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;

// bf16 word -> fp32 (exact).
__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 word, round to nearest even; NaN -> 0x7fc0. This is bit-for-bit the conversion of
// torch's c10::BFloat16 (and of a plain IEEE RNE narrowing for every non-NaN input).
__device__ __forceinline__ uint32_t f2bf_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two fp32 -> one dword of two bf16 (lo in bits 0..15) with one v_cvt_pk_bf16_f32 (round to nearest
// even). Used where values are finite by construction (softmax weights, outputs).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}
// The gated MLP activation on two bf16 pairs (serve/fast_kernels.py:526-545, _silu_mul_kernel): the gate's
// SiLU rounded to bf16 first (act(gate) in bf16, as the model's MLP), then times up, rounded again. Shared by
// k_silu_mul and the w13 GEMM's gated epilogue, so the fused and separate paths give the same bits. The SiLU is
// g * rcp(1 + 2^(-g log2 e)) on the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32, about 1 ulp each; the
// reference's tl.exp is an approximate exp as well): its result is rounded to bf16 at once, which these errors
// move only where a value lies within ~2^-16 of a bf16 rounding boundary. Large negative g: 2^(...) = inf,
// rcp(inf) = 0, g * 0 = -0, as g / inf. (A full-precision expf and an IEEE divide cost ~4x the VALU
// instructions, about 1.8 us of the w13 epilogue at 192 x 4864.)
__device__ __forceinline__ float silu_f32(float g) {
  return g * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * g));
}
__device__ __forceinline__ uint32_t silu_mul_bf16x2(uint32_t g2, uint32_t u2) {
  const float g0 = bf_lo(g2), g1 = bf_hi(g2);
  const uint32_t gs = pack_bf16x2(silu_f32(g0), silu_f32(g1));
  return pack_bf16x2(bf_lo(gs) * bf_lo(u2), bf_hi(gs) * bf_hi(u2));
}

__device__ __forceinline__ u32x4 ld16(const void *p) { return *reinterpret_cast<const u32x4 *>(p); }
// 16-byte LDS read (ds_read_b128) from a generic pointer known to point into LDS.
__device__ __forceinline__ u32x4 lds_ld16(const void *p) {
  return *(const __attribute__((address_space(3))) u32x4 *)const_cast<void *>(p);
}
__device__ __forceinline__ void st16(void *p, u32x4 v) { *reinterpret_cast<u32x4 *>(p) = v; }
__device__ __forceinline__ void st8(void *p, u32x2 v) { *reinterpret_cast<u32x2 *>(p) = v; }

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// Raw buffer resource over [base, base + bytes): loads at byte offsets >= bytes return zeros without
// touching memory (the descriptor's range check), which is how the kernels mask key rows past a range
// and prefetch past its end. Word 3 = 0x00020000 is the gfx9-family raw-buffer format.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
// The same descriptor from a base and size the compiler cannot prove wave-uniform (values derived from
// vector-loaded metadata): reading them from the first lane makes the descriptor scalar, where a
// divergent descriptor would wrap every load in a loop over lanes.
__device__ __forceinline__ rsrc_t make_rsrc_wave(const void *base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return make_rsrc(reinterpret_cast<const void *>(((uint64_t)hi << 32) | lo), __builtin_amdgcn_readfirstlane(bytes));
}
// Partials exchanged between the workgroups of one launch (the in-kernel merges): a partial goes out with
// agent-coherent (sc1) buffer stores, which write through the XCD's L2; once they have completed (vmcnt(0))
// an atomic on the unit's counter makes the arrival known, and the last arrival reads every partial with sc1
// loads issued after its atomic returned. Only the bytes exchanged are kept coherent: an agent-scope fence
// would write back and invalidate the whole L2 for every partial, under the other workgroups' loads.
constexpr int kSC1 = 16;  // buffer cache policy: sc1, coherent across the device (agent scope)
// 4-byte vector-memory load at byte offset `off`. Unlike a scalar load of a uniform address, it is
// counted with the tile loads (vmcnt), so waiting for it never waits for the LDS traffic or vice versa.
__device__ __forceinline__ int bld4(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
// 16-byte load at byte offset `off` (the whole offset in the VGPR operand, so the range check sees it).
__device__ __forceinline__ u32x4 bld16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// 16-byte-per-lane DMA from a raw buffer straight into LDS (buffer_load_dwordx4 ... lds): lane l's
// 16 bytes from buffer offset voff + soff + IMM land at LDS address lds + IMM + 16 l (the immediate
// moves both sides, soff only the buffer side). The range check covers voff + soff + IMM; lanes past
// the range write zeros. lds must be wave-uniform (it goes to M0). Completion is counted in vmcnt.
// CPOL: the instruction's cache-policy bits (2 = nt: non-temporal, for data read once).
typedef __attribute__((address_space(3))) void lds_void_t;
template <int IMM, int CPOL = 0>
__device__ __forceinline__ void bld16_lds(rsrc_t r, void *lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)lds, 16, voff, soff, IMM, CPOL);
}

// s_waitcnt vmcnt(N), expcnt and lgkmcnt left at their maxima: at most N of this wave's vector-memory
// operations (loads, stores, LDS DMA) still outstanding. They complete in issue order, so an operation is
// done once N others are known to have been issued after it. Every read of LDS written by DMA waits this
// way, with N counted at the call site: the compiler's own wait for LDS DMA has been seen missing (no
// wait at all before the reads at a loop's head, for DMA issued in the previous iteration).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// ds_read_b64_tr_b16: within each 16-lane group, lane i supplies the address of 4 consecutive bf16 and
// lane j receives, in slot k, element j%4 of lane 4k + j/4's data. With lane i pointing at row
// (r0 + i/4), columns c0 + 4(i%4).. of a row-major bf16 matrix, lane j receives column c0 + j of rows
// r0..r0+3: a 4 x 16 block read transposed.
typedef short i16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_tr16(const void *p) {
  return __builtin_bit_cast(
      u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4 *)const_cast<void *>(p)));
}

// D = A(16x32) * B(32x16) + C, bf16 in, fp32 accumulate. Lane l supplies A[l%16][8*(l/16)+j] and
// B[8*(l/16)+j][l%16] (j = 0..7) and receives D[4*(l/16)+i][l%16] (i = 0..3). Only the pairing of A
// and B slots matters for the sum over k, so callers may map any 32 reduction indices onto the
// (lane group, slot) pairs as long as A and B use the same map.
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max(a, b, c) as one v_maximum3_f32 (IEEE 754-2019 maximum: a NaN input gives NaN). fmaxf() on values
// the compiler cannot prove canonical (MFMA results) first quiets each input with a v_max x, x of its own;
// maximum needs no quieting. Written with the builtin (not asm) so the compiler still inserts the wait
// states between an MFMA and a VALU read of its result.
__device__ __forceinline__ float max3_ieee(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
__device__ __forceinline__ float max_ieee(float a, float b) { return __builtin_elementwise_maximum(a, b); }
// max_over_groups with maximum instead of fmaxf
__device__ __forceinline__ float max_over_groups_ieee(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = max_ieee(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return max_ieee(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Cross-lane reductions over the four 16-lane groups of a wave (lanes l, l^16, l^32, l^48), with the
// gfx950 lane swaps (VALU, no LDS round trip): v_permlane16_swap(v, v) yields the values of the even and
// the odd 16-lane row of each row pair, v_permlane32_swap(v, v) those of the lower and the upper 32
// lanes, so one swap plus one operation reduces over l, l^16 and a second over l, l^32. Every lane of a
// set gets the same bits.
__device__ __forceinline__ float max_over_groups(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_over_groups(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Orders LDS traffic between the lanes of one wave: the hardware serves one wave's LDS
// instructions in issue order, so only the compiler's reordering has to be stopped.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Workgroup barrier for data exchanged through LDS with ordinary LDS stores: compiler-only fences,
// this wave's LDS operations completed (s_waitcnt lgkmcnt(0)), then s_barrier. Vector-memory loads
// and LDS DMA stay in flight: __syncthreads() would wait for all of them (on gfx9 one counter tracks
// loads and stores, and its fence covers LDS DMA), draining the loads prefetched for the next tiles.
// Not for LDS written by DMA.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Four 16-byte LDS stores at byte offsets 0, 64, 128, 192 from p. Written as one asm block because
// the compiler's wait bookkeeping may take plain stores next to in-flight LDS DMA as overlapping it
// and drain every outstanding load first. Completion is not tracked: wait with lds_barrier (or an
// explicit lgkmcnt(0)) before the data is read.
__device__ __forceinline__ void lds_store_4x16(void *p, f32x4 a, f32x4 b, f32x4 c, f32x4 d) {
  const uint32_t addr = (uint32_t)reinterpret_cast<uintptr_t>(p);
  asm volatile(
      "ds_write_b128 %0, %1\n\t"
      "ds_write_b128 %0, %2 offset:64\n\t"
      "ds_write_b128 %0, %3 offset:128\n\t"
      "ds_write_b128 %0, %4 offset:192"
      :
      : "v"(addr), "v"(a), "v"(b), "v"(c), "v"(d)
      : "memory");
}

// Brings the first BYTES of the kernel's argument block into the scalar cache with one batch of loads
// (one per 64-byte line, all in flight together). The compiler fetches arguments where they are first
// needed, in several dependent rounds around early branches and barriers; each round is a scalar-cache
// miss to L2 and together they held the first memory requests of a launch back by ~2 us. BYTES must not
// exceed the explicit arguments' size.
template <int BYTES>
__device__ __forceinline__ void warm_kernargs() {
  const uint32_t *p = (const uint32_t *)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t acc = 0;
#pragma unroll
  for (int o = 0; o < BYTES; o += 64) acc += p[o / 4];
  asm volatile("" : : "s"(acc));
}

// LDS words of a handshake between the waves of a workgroup, as asm for the same reason. Each waits
// for the wave's earlier LDS operations first (so they are visible to any wave that sees the new word)
// and returns with its own operation complete.
// lds_add_word: adds v of lane 0 (the other lanes add 0) and returns, in every lane, the word before it.
__device__ __forceinline__ int lds_add_word(int *p, int v) {
  const uint32_t addr = (uint32_t)reinterpret_cast<uintptr_t>(p);
  const int mine = (__lane_id() == 0) ? v : 0;
  int r;
  asm volatile("s_waitcnt lgkmcnt(0)\n\tds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
               : "=v"(r)
               : "v"(addr), "v"(mine)
               : "memory");
  return __builtin_amdgcn_readlane(r, 0);
}
__device__ __forceinline__ int lds_read_word(const int *p) {
  const uint32_t addr = (uint32_t)reinterpret_cast<uintptr_t>(p);
  int r;
  asm volatile("s_waitcnt lgkmcnt(0)\n\tds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(addr) : "memory");
  return __builtin_amdgcn_readfirstlane(r);
}
__device__ __forceinline__ void lds_write_word(int *p, int v) {
  const uint32_t addr = (uint32_t)reinterpret_cast<uintptr_t>(p);
  asm volatile("s_waitcnt lgkmcnt(0)\n\tds_write_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : : "v"(addr), "v"(v) : "memory");
}

// 8x8 transpose of bf16 words held as 8 rows x 16 bytes: out[c] collects element c of every row
// (row j in slot j). Each output dword pairs rows (2e, 2e+1).
__device__ __forceinline__ void transpose8x8_bf16(const u32x4 (&in)[8], u32x4 (&out)[8]) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int dw = c >> 1;
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t a = in[2 * e][dw], b = in[2 * e + 1][dw];
      o[e] = (c & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
    }
    out[c] = o;
  }
}

// Records the message for a negative status on the calling host thread and returns `code`
// (defined in capi.hip).
int set_error(int code, const char *fmt, ...);

// The generic-head decode kernel (attn_cols.hip) for head_dim 128, behind the decode entry points (which check
// their arguments first).
int attn_cols_decode(const char *fn, const void *q, int64_t s_qb, int64_t s_qh, const void *kc, const void *vc,
                     int64_t s_kb, int64_t s_kh, int cache_rows, int cache_len, const int32_t *lens,
                     const int32_t *rowmap, void *out, int64_t s_ob, int64_t s_oh, int b, int nq, int nkv, int hd,
                     float scale, hipStream_t stream);
// The head_dim-128 packed prefill (prefill128.hip), behind a8_prefill_attn (which checks its arguments first).
int prefill128(const void *q, int64_t s_qr, int64_t s_qh, int R, const void *kc, const void *vc, int64_t s_kb,
               int64_t s_kh, int cache_rows, int cache_len, void *out, int64_t s_or, int64_t s_oh, const int32_t *bq0,
               const int32_t *bn, const int32_t *bslot, const int32_t *bpos0, int nblk, int nq, int group,
               float scale, hipStream_t stream);

}  // namespace a8
