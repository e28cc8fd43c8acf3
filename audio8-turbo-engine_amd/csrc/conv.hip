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
// MI355X design (an implicit GEMM: M = B*TR rows, N = Cout, K = TAPS*Cin): a workgroup computes a BM x BN
// output tile of one phase (BM = 64 WM rows, BN = 16 NT channels, up to 128 x 256) with 4 waves, each wave
// WM row tiles of 16 x BN on v_mfma_f32_16x16x32_f16, as Y^T = W^T . X^T:
//   * X rows are the B operands straight from global memory (lane l: 16 contiguous bytes of row l % 16 at
//     channel offset 8 (l / 16)), with the snake applied in registers;
//   * each KS x BN weight slice [k][n] (KS = 64 channels, else 96, else 32, whichever divides Cin) is staged
//     once in LDS and read as the A operand with ds_read_b64_tr_b16
//     (the LDS unit transposes 4 x 16 blocks), so W^T needs no copy;
//     one A operand feeds WM MFMAs;
//   * two LDS slice areas filled by DMA (buffer_load ... lds), the next slice's DMA and X loads issued
//     right after the barrier that frees its area, before the current slice's MFMAs; one barrier a slice
//     and no register copies between steps;
//   * the tile shape is chosen per launch (conv_plan): the fewest padded output channels, then, among shapes
//     that give >= 512 workgroups, two row tiles per wave and the widest tile; narrow tiles for short inputs;
//   * short inputs with long K (the decoder's first blocks: a few hundred rows x 5-7 K channels) split K
//     over workgroups into an fp32 workspace the caller provides (a8_conv_cl_ws_bytes), summed in a fixed
//     order by a finishing kernel, so results do not depend on timing.
// The snake's sine runs on the hardware sine unit after an exact reduction to one period.
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
// sin(x) on the hardware sine (v_sin_f32 takes revolutions): x / 2 pi reduced to [-1/2, 1/2] by its nearest
// integer, so the unit sees its most accurate range; absolute error ~1e-6 for the snake's |a x| < 100, far
// below the fp16 rounding of the result
__device__ __forceinline__ float sin_hw(float x) {
  float r = x * 0.15915494309189535f;
  r -= __builtin_rintf(r);
  return __builtin_amdgcn_sinf(r);
}
__device__ __forceinline__ u32x2 ld8(const void *p) { return *reinterpret_cast<const u32x2 *>(p); }
// the snake x + ib sin(a x)^2 on 8 channels (fp32, one rounding to fp16). No contraction: left free, the compiler
// fuses the last add and the fp16 conversion into one v_fma_mix at some call sites and not at others (one
// rounding against two), and the same row would get different bits in snake_cat, the conv loads and the state.
__device__ __forceinline__ u32x4 snake8(u32x4 v, const float *a, const float *ib) {
#pragma clang fp contract(off)
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float x0 = h_lo(v[j]), x1 = h_hi(v[j]);
    const float s0 = sin_hw(x0 * a[2 * j]), s1 = sin_hw(x1 * a[2 * j + 1]);
    o[j] = pack_f16x2(x0 + ib[2 * j] * s0 * s0, x1 + ib[2 * j + 1] * s1 * s1);
  }
  return o;
}

constexpr int kSnakeMaxC = 1024;  // input channels a conv with the snake on its loads may have

// RU: a whole residual unit (the reference's ru_fused, serve/fast_kernels.py:626-692), the 1x1 conv in the
// k-tap conv's epilogue: h = acc + bias (fp32), snake with a2 / ib2 (fp32, one fp16 rounding), then
// out = h' . w2 + b2 + res. Needs the whole channel width in one tile (Cout = BN, one column tile).
template <int WM, int NT, int KSUB, bool SNAKE, bool RU = false>
__global__ __launch_bounds__(256, 2) void k_conv_cl(const uint16_t *__restrict__ x, int64_t s_xb, int64_t s_xt,
                                                 const uint16_t *__restrict__ w, int64_t s_wp, int64_t s_wt,
                                                 int64_t s_wc, const uint16_t *__restrict__ bias,
                                                 const uint16_t *__restrict__ res, int64_t s_rb, int64_t s_rt,
                                                 uint16_t *__restrict__ y, int64_t s_yb, int64_t s_yt,
                                                 const float *__restrict__ sa, const float *__restrict__ sib, int M,
                                                 int TR, int Cin, int Cout, int CoutW, int taps, int dil, int PH,
                                                 float *__restrict__ part, int ksplit, uint32_t x_span,
                                                 uint32_t w_span, const uint16_t *__restrict__ w2,
                                                 const uint16_t *__restrict__ b2, const float *__restrict__ a2,
                                                 const float *__restrict__ ib2, uint32_t w2_span) {
  warm_kernargs<220>();  // the explicit arguments above span 0x00-0xdb
  static_assert(!RU || (!SNAKE && NT % 2 == 0), "residual unit: input pre-activated, 32-channel k steps");
  constexpr int BN = 16 * NT, BM = 64 * WM, KS = 32 * KSUB, NCH = BN / 8;
  // two weight slices [k][n] (KS x BN): one is read while the next is written. A k row is BN + 16 elements
  // apart: the 16 rows one transposing read touches then fall on distinct bank groups (at a pitch of BN,
  // a multiple of 64 elements, they all hit the same 8 banks: 4x the LDS cycles, measured as bank conflicts)
  constexpr int BNP = BN + 16;
  // A slice goes from memory into LDS by DMA (buffer_load ... lds: one instruction fills 64 consecutive
  // 16-byte chunks): chunk c of a slice is k row c / RC, column chunk c % RC, the last two chunks of a row
  // being the padding. Each wave issues R instructions a slice, so the slice area is rounded up to R * 256
  // chunks (the chunks past the slice and the padding receive zeros). Two slice areas as two arrays: the
  // compiler then tells their DMA completions apart.
  constexpr int RC = NCH + 2, R = (KS * RC + 255) / 256, SL = R * 256 * 8;
  __shared__ __attribute__((aligned(16))) uint16_t wlA[SL];
  __shared__ __attribute__((aligned(16))) uint16_t wlB[SL];
  const int p = blockIdx.z / ksplit, ks = blockIdx.z - p * ksplit, m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  // Operand loads are buffer loads with the range check as the mask (an invalid lane asks for offset
  // kOob and reads zeros): no branch around a load, so the compiler's wait before the MFMAs covers only
  // the operands they use, not the next slice's loads in flight (conditional loads made it vmcnt(0)).
  constexpr uint32_t kOob = 0x80000000u;  // the entry point checks both spans are below it
  const rsrc_t xr = make_rsrc(x, x_span), wr = make_rsrc(w, w_span);
  // this lane's X rows (the B operands' column r16 of the wave's WM row tiles) and channel chunk 8g
  uint32_t xoff[WM];
  int mb[WM], mt[WM];
  bool mv[WM];
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int m = m0 + (wv * WM + i) * 16 + r16;
    mv[i] = m < M;
    mb[i] = mv[i] ? m / TR : 0;
    mt[i] = mv[i] ? m - mb[i] * TR : 0;
    xoff[i] = (uint32_t)(((int64_t)mb[i] * s_xb + (int64_t)mt[i] * s_xt + 8 * g) * 2);
  }
  // this lane's chunk of each of the wave's R DMA instructions: c = (4 r + wave) 64 + lane
  int wk[R];
  uint32_t wb[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int c = (4 * r + wv) * 64 + lane, kr = c / RC, cc = c - kr * RC;
    const bool ok = kr < KS && cc < NCH && n0 + 8 * cc < CoutW;
    wk[r] = ok ? kr : Cin;  // a chunk that is never valid gets a k row past every slice
    wb[r] = ok ? (uint32_t)(((int64_t)p * s_wp + (int64_t)kr * s_wc + n0 + 8 * cc) * 2) : 0u;
  }
  // this workgroup's k slices: [sb, se) of taps * ceil(Cin / KS) (a 1 / ksplit share under split-K)
  const int kchunks = (Cin + KS - 1) / KS, steps = taps * kchunks;
  const int sb = (int)((int64_t)steps * ks / ksplit), se = (int)((int64_t)steps * (ks + 1) / ksplit);

  // slice s of the weights into LDS area dst (the slice's uniform offset goes in soffset)
  auto issue_w = [&](int s, uint16_t *dst) __attribute__((always_inline)) {
    const int j = s / kchunks, k0 = (s - j * kchunks) * KS;
    const uint32_t so = (uint32_t)(((int64_t)j * s_wt + (int64_t)k0 * s_wc) * 2);
#pragma unroll
    for (int r = 0; r < R; ++r)
      bld16_lds<0>(wr, dst + (4 * r + wv) * 512, k0 + wk[r] < Cin ? wb[r] : kOob, so);
  };
  auto load_x = [&](int s, int i, int u) __attribute__((always_inline)) -> u32x4 {
    const int j = s / kchunks, k0 = (s - j * kchunks) * KS + 32 * u;
    const bool ok = mv[i] && k0 + 8 * g < Cin;
    return bld16(xr, ok ? xoff[i] + (uint32_t)(((int64_t)j * dil * s_xt + k0) * 2) : kOob);
  };
  // The snake runs where an operand is used, not where it is loaded (applied at the load it would wait
  // for the load at once and undo the prefetch); its vectors are staged in LDS once per workgroup
  // (visible after the first step's barrier).
  __shared__ __attribute__((aligned(16))) float sabl[SNAKE ? 2 * kSnakeMaxC : 4];
  if (SNAKE)
    for (int c = tid; c < Cin; c += 256) {
      sabl[c] = sa[c];
      sabl[kSnakeMaxC + c] = sib[c];
    }
  auto operand = [&](u32x4 v, int s, int u) __attribute__((always_inline)) -> u32x4 {
    if (!SNAKE) return v;
    const int j = s / kchunks, k0 = (s - j * kchunks) * KS + 32 * u;
    // snake(0) = 0: lanes that read zeros stay zero, so their snake vectors may be any in-range entries
    const int kc = k0 + 8 * g < Cin ? k0 + 8 * g : 0;
    float a[8], ib[8];
    const f32x4 a0 = *reinterpret_cast<const f32x4 *>(sabl + kc), a1 = *reinterpret_cast<const f32x4 *>(sabl + kc + 4);
    const f32x4 i0 = *reinterpret_cast<const f32x4 *>(sabl + kSnakeMaxC + kc);
    const f32x4 i1 = *reinterpret_cast<const f32x4 *>(sabl + kSnakeMaxC + kc + 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      a[q] = a0[q];
      a[4 + q] = a1[q];
      ib[q] = i0[q];
      ib[4 + q] = i1[q];
    }
    return snake8(v, a, ib);
  };

  f32x4 acc[WM][NT];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[i][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  // A-operand reads: rows (k) 8g + r16/4 (+4), columns (n) 16 nt + 4 (r16 % 4)
  const int aoff = (8 * g + (r16 >> 2)) * BNP + 4 * (r16 & 3);
  u32x4 xa[WM][KSUB], xb[WM][KSUB];
  issue_w(sb, wlA);
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int u = 0; u < KSUB; ++u) xa[i][u] = load_x(sb, i, u);
  // One k slice s, its weights in `cur` (DMA issued one step earlier) and its X operands in xc (loaded one
  // step earlier): wait for this wave's DMA of the slice (the X loads issued after it may still fly), the
  // barrier (every wave's DMA landed; every wave is done with `nxt`, slice s - 1), the DMA of slice s + 1
  // into `nxt` and its X loads into xn (the last step reloads its own slice: no branch), then the MFMAs.
  // No register copies between steps: loads stay in flight until their first use.
  auto step = [&](int s, u32x4(&xc)[WM][KSUB], u32x4(&xn)[WM][KSUB], const uint16_t *cur,
                  uint16_t *nxt) __attribute__((always_inline)) {
    constexpr int nx = WM * KSUB;  // X loads issued after a slice's DMA
    static_assert(nx < 16, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt(0x0F70 | nx);  // s_waitcnt vmcnt(nx)
    __syncthreads();
    const int s1 = s + 1 < se ? s + 1 : s;
    issue_w(s1, nxt);
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int u = 0; u < KSUB; ++u) xn[i][u] = load_x(s1, i, u);
#pragma unroll
    for (int u = 0; u < KSUB; ++u) {
      u32x4 xo[WM];
#pragma unroll
      for (int i = 0; i < WM; ++i) xo[i] = operand(xc[i][u], s, u);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const uint16_t *ap = cur + aoff + 32 * u * BNP + 16 * nt;
        const u32x2 lo = lds_tr16(ap), hi = lds_tr16(ap + 4 * BNP);
        const u32x4 a = u32x4{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int i = 0; i < WM; ++i) acc[i][nt] = mfma16x16x32_f16(a, xo[i], acc[i][nt]);
      }
    }
  };
  int s = sb;
  for (; s + 1 < se; s += 2) {
    step(s, xa, xb, wlA, wlB);
    step(s + 1, xb, xa, wlB, wlA);
  }
  if (s < se) step(s, xa, xb, wlA, wlB);
  // the DMA issued by the last step (its own slice again) still writes LDS: let it land before the
  // workgroup ends. s_waitcnt vmcnt(0).
  __builtin_amdgcn_s_waitcnt(0x0F70);
  if constexpr (RU) {
    // Residual unit, second conv (1x1, k = Cout = BN channels) on the first one's output, in registers.
    // h = acc + bias, then the snake (fp32, one rounding to fp16), packed straight into the 1x1's B
    // operands: slot 8g + j of 32-channel step u holds channel 32u + 16 (j / 4) + 4g + j % 4 -- where this
    // lane's accumulators already are (acc[i][2u], acc[i][2u + 1]); the A operands read w2 in the same
    // channel order (rows 4g.. and 16 + 4g.. of each 32-row block). No data moves between lanes.
    constexpr int KU = NT / 2;
    u32x4 hb[WM][KU];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int n = 16 * nt + 4 * g;
      const u32x2 bv = ld8(bias + n);
      const f32x4 av = *reinterpret_cast<const f32x4 *>(a2 + n), iv = *reinterpret_cast<const f32x4 *>(ib2 + n);
      const float bb[4] = {h_lo(bv[0]), h_hi(bv[0]), h_lo(bv[1]), h_hi(bv[1])};
#pragma unroll
      for (int i = 0; i < WM; ++i) {
        float hv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float h = acc[i][nt][e] + bb[e];
          const float sv = sin_hw(h * av[e]);
          hv[e] = h + iv[e] * sv * sv;
        }
        hb[i][nt >> 1][2 * (nt & 1)] = pack_f16x2(hv[0], hv[1]);
        hb[i][nt >> 1][2 * (nt & 1) + 1] = pack_f16x2(hv[2], hv[3]);
        acc[i][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    // w2 [k][n] (row pitch s_wc, as w's) through the same two LDS slice areas, KS rows a slice; every wave
    // is done with them once it passes the barrier (its last slice's reads are in its accumulators)
    const rsrc_t w2r = make_rsrc(w2, w2_span);
    auto issue_w2 = [&](int s2, uint16_t *dst) __attribute__((always_inline)) {
      const int k0 = s2 * KS;
      const uint32_t so = (uint32_t)((int64_t)k0 * s_wc * 2);
#pragma unroll
      for (int r = 0; r < R; ++r)
        bld16_lds<0>(w2r, dst + (4 * r + wv) * 512, k0 + wk[r] < Cin ? wb[r] : kOob, so);  // (p = 0, n0 = 0)
    };
    const int aoff2 = (4 * g + (r16 >> 2)) * BNP + 4 * (r16 & 3);
    constexpr int S2 = BN / KS;  // the host launches RU only where KS divides BN
    static_assert(BN % KS == 0, "1x1 slices");
    __syncthreads();
    issue_w2(0, wlA);
#pragma unroll
    for (int s2 = 0; s2 < S2; ++s2) {
      uint16_t *cur = (s2 & 1) ? wlB : wlA, *nxt = (s2 & 1) ? wlA : wlB;
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's DMA of slice s2
      __syncthreads();                     // every wave's; every wave is done with nxt
      if (s2 + 1 < S2) issue_w2(s2 + 1, nxt);
#pragma unroll
      for (int u = 0; u < KSUB; ++u) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const uint16_t *ap = cur + aoff2 + 32 * u * BNP + 16 * nt;
          const u32x2 lo = lds_tr16(ap), hi = lds_tr16(ap + 16 * BNP);
          const u32x4 a = u32x4{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
          for (int i = 0; i < WM; ++i) acc[i][nt] = mfma16x16x32_f16(a, hb[i][s2 * KSUB + u], acc[i][nt]);
        }
      }
    }
    bias = b2;  // the epilogue below adds the second conv's bias and the unit's input
  }
  // acc[i][nt]: lane (r16, g) holds Y[row m0 + (wv WM + i) 16 + r16][n = n0 + 16 nt + 4g + e], e = 0..3
  if (part) {  // split-K: raw fp32 sums to part[ks][p][m][n], row pitch gridDim.y BN; k_conv_fin finishes
    const int64_t NP = (int64_t)gridDim.y * BN;
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      if (!mv[i]) continue;
      float *prow = part + ((int64_t)(ks * PH + p) * M + m0 + (wv * WM + i) * 16 + r16) * NP + n0 + 4 * g;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) *reinterpret_cast<f32x4 *>(prow + 16 * nt) = acc[i][nt];
    }
    return;
  }
  // bias and residual by 8-byte loads where four channels share them (uniform)
  const bool vec = (Cout & 3) == 0 && (reinterpret_cast<uintptr_t>(bias) & 7u) == 0 &&
                   (reinterpret_cast<uintptr_t>(y) & 7u) == 0 && ((s_yb | s_yt) & 3) == 0 &&
                   (!res || ((reinterpret_cast<uintptr_t>(res) & 7u) == 0 && ((s_rb | s_rt) & 3) == 0));
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    if (!mv[i]) continue;
    const int64_t orow = (int64_t)mt[i] * PH + p;
    uint16_t *yrow = y + (int64_t)mb[i] * s_yb + orow * s_yt;
    const uint16_t *rrow = res ? res + (int64_t)mb[i] * s_rb + orow * s_rt : nullptr;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int n = n0 + 16 * nt + 4 * g;
      if (n >= Cout) continue;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = acc[i][nt][e];
      if (vec) {  // n + 3 < Cout
        if (bias) {
          const u32x2 bv = ld8(bias + n);
          v[0] += h_lo(bv[0]), v[1] += h_hi(bv[0]), v[2] += h_lo(bv[1]), v[3] += h_hi(bv[1]);
        }
        if (rrow) {
          const u32x2 rv = ld8(rrow + n);
          v[0] += h_lo(rv[0]), v[1] += h_hi(rv[0]), v[2] += h_lo(rv[1]), v[3] += h_hi(rv[1]);
        }
        st8(yrow + n, u32x2{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])});
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (n + e >= Cout) continue;
          if (bias) v[e] += h_lo(bias[n + e]);
          if (rrow) v[e] += h_lo(rrow[n + e]);
          yrow[n + e] = (uint16_t)(pack_f16x2(v[e], 0.f) & 0xffffu);
        }
      }
    }
  }
}

// Split-K finish: Y = sum over ks of part[ks] (in ks order) + bias (+ res), one rounding to fp16; one thread per
// 4 channels of one output row.
__global__ __launch_bounds__(256) void k_conv_fin(const float *__restrict__ part, int64_t NP, int ksplit,
                                                  const uint16_t *__restrict__ bias, const uint16_t *__restrict__ res,
                                                  int64_t s_rb, int64_t s_rt, uint16_t *__restrict__ y, int64_t s_yb,
                                                  int64_t s_yt, int M, int TR, int Cout, int PH) {
  warm_kernargs<92>();  // the explicit arguments above span 0x00-0x5b
  const int nq = (Cout + 3) >> 2;
  const uint32_t id = blockIdx.x * 256u + threadIdx.x;
  if (id >= (uint32_t)PH * (uint32_t)M * (uint32_t)nq) return;
  const int c = (int)(id % (uint32_t)nq);
  const uint32_t pm = id / (uint32_t)nq;
  const int m = (int)(pm % (uint32_t)M), p = (int)(pm / (uint32_t)M), n = 4 * c;
  f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < ksplit; ++k) v += *reinterpret_cast<const f32x4 *>(part + ((int64_t)(k * PH + p) * M + m) * NP + n);
  const int b = m / TR, t = m - b * TR;
  const int64_t orow = (int64_t)t * PH + p;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (n + e >= Cout) continue;
    float o = v[e];
    if (bias) o += h_lo(bias[n + e]);
    if (res) o += h_lo(res[(int64_t)b * s_rb + orow * s_rt + n + e]);
    y[(int64_t)b * s_yb + orow * s_yt + n + e] = (uint16_t)(pack_f16x2(o, 0.f) & 0xffffu);
  }
}

template <bool SNAKE, bool REFRESH>
__global__ __launch_bounds__(256) void k_snake_cat(const uint16_t *__restrict__ x, int64_t s_xb, int64_t s_xt,
                                                   uint16_t *st, int64_t s_sb, int64_t s_st,
                                                   const float *__restrict__ sa, const float *__restrict__ sib,
                                                   uint16_t *__restrict__ y, int64_t s_yb, int64_t s_yt, int B,
                                                   int T, int CTX, int C) {
  warm_kernargs<104>();  // the explicit arguments above span 0x00-0x67
  const int nch = C >> 3;
  // REFRESH (T >= CTX): one item per x row j; item j < CTX also moves state row j into y and writes the new
  // state row j (y's row T + j = snake(x[T - CTX + j])) after reading the old one -- the only reader of that row
  const int rows = REFRESH ? T : CTX + T;
  const uint32_t id = blockIdx.x * 256u + threadIdx.x;
  if (id >= (uint32_t)B * (uint32_t)rows * (uint32_t)nch) return;
  const int c = (int)(id % (uint32_t)nch);
  const uint32_t rt = id / (uint32_t)nch;
  const int tt = (int)(rt % (uint32_t)rows), b = (int)(rt / (uint32_t)rows);
  float a[8], ib[8];
  if (SNAKE) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      a[q] = sa[8 * c + q];
      ib[q] = sib[8 * c + q];
    }
  }
  auto act = [&](int j) {
    u32x4 v = ld16(x + (int64_t)b * s_xb + (int64_t)j * s_xt + 8 * c);
    return SNAKE ? snake8(v, a, ib) : v;
  };
  if (REFRESH) {
    st16(y + (int64_t)b * s_yb + (int64_t)(CTX + tt) * s_yt + 8 * c, act(tt));
    if (tt < CTX) {
      uint16_t *sp = st + (int64_t)b * s_sb + (int64_t)tt * s_st + 8 * c;
      const u32x4 old = ld16(sp);
      st16(y + (int64_t)b * s_yb + (int64_t)tt * s_yt + 8 * c, old);
      st16(sp, act(T - CTX + tt));
    }
    return;
  }
  const u32x4 v = tt < CTX ? ld16(st + (int64_t)b * s_sb + (int64_t)tt * s_st + 8 * c) : act(tt - CTX);
  st16(y + (int64_t)b * s_yb + (int64_t)tt * s_yt + 8 * c, v);
}

// The decoder's last conv (one output channel) with everything around it (a8_conv_out_tanh): snake_cat's
// [state | snake(x)], the causal conv of `taps` taps (dilation 1) into one channel with fp32 sums, the fp16
// rounding conv_cl would store, then tanh in fp32 (serve/fast_engine.py:228-233 and 310: snake_cat, conv_cl,
// the state refresh, y[..., 0].float().tanh()). Workgroup (b, tb) computes outputs t = kCoT tb .. + kCoT - 1 of row
// b from the activated rows t .. t + taps - 1 of [state | snake(x)] staged in LDS; workgroup (b, 0), the only
// one reading row b's old state, also writes the new state (the last CTX activated rows, T >= CTX) after its
// staging has read the old one. The products run on MFMA with the taps as columns: Z[r][j] = A[r] . w[j] for
// every staged row r (v_mfma_f32_16x16x32_f16, 16 rows x 32 channels x the taps padded to 16 columns), then
// y[t] = sum_j Z[t + j][j] in fp32 in tap order. Graph-replayed at 192 x 2048 x 96: 25.9 us, against 45.1 us
// for a dot product per output on the VALU (every operand converted for every tap); conv_cl's implicit GEMM
// pads the one column to 16. Each thread requests all of its staged rows before any snake (one round trip),
// and 128 outputs a workgroup fit four workgroups per compute unit (256: 32.0 us, 64: 25.4 us).
#ifndef A8_CO_T
#define A8_CO_T 128
#endif
constexpr int kCoT = A8_CO_T;    // outputs per workgroup (the staged rows then fit four workgroups per compute unit)
constexpr int kCoMaxCin = 128;   // input channels (the decoder's last block has 96)
constexpr int kCoMaxTaps = 8;
constexpr int kCoPitch = kCoMaxCin + 8;  // LDS row pitch (elements): consecutive rows start 4 banks apart

__global__ __launch_bounds__(256) void k_conv_out(const uint16_t *__restrict__ x, int64_t s_xb, int64_t s_xt,
                                                  uint16_t *st, int64_t s_sb, int64_t s_st,
                                                  const float *__restrict__ sa, const float *__restrict__ sib,
                                                  const uint16_t *__restrict__ w, const uint16_t *__restrict__ bias,
                                                  float *__restrict__ y, int64_t s_yb, int T, int CTX, int Cin,
                                                  int taps) {
  warm_kernargs<104>();  // the explicit arguments above span 0x00-0x67
  __shared__ __attribute__((aligned(16))) uint16_t xs[(kCoT + kCoMaxTaps) * kCoPitch];
  __shared__ __attribute__((aligned(16))) uint16_t ws[kCoMaxTaps * kCoMaxCin];
  __shared__ float a_s[kCoMaxCin], ib_s[kCoMaxCin];
  const int nt = (T + kCoT - 1) / kCoT;
  const int b = blockIdx.x / nt, tb = blockIdx.x - b * nt;
  const int t0 = tb * kCoT, tid = threadIdx.x;
  const int nch = Cin >> 3;
  for (int i = tid; i < taps * nch; i += 256) st16(ws + 8 * i, ld16(w + 8 * i));
  for (int i = tid; i < Cin; i += 256) {
    a_s[i] = sa[i];
    ib_s[i] = sib[i];
  }
  __syncthreads();
  // rows q = t0 .. t0 + kCoT + taps - 2 of [state | snake(x)] (q < CTX: the state's row q, else x's row q - CTX)
  const int nrow = min(kCoT, T - t0) + taps - 1;
  const uint16_t *xb = x + (int64_t)b * s_xb;
  uint16_t *sb = st + (int64_t)b * s_sb;
  // every load of this thread first, then the snake and the LDS stores (one round trip, not one per row)
  constexpr int kCoIt = ((kCoT + kCoMaxTaps) * (kCoMaxCin / 8) + 255) / 256;
  u32x4 v[kCoIt];
#pragma unroll
  for (int it = 0; it < kCoIt; ++it) {
    const int i = tid + 256 * it;
    if (i >= nrow * nch) break;
    const int r = i / nch, c = i - r * nch, q = t0 + r;
    v[it] = ld16(q < CTX ? sb + (int64_t)q * s_st + 8 * c : xb + (int64_t)(q - CTX) * s_xt + 8 * c);
  }
#pragma unroll
  for (int it = 0; it < kCoIt; ++it) {
    const int i = tid + 256 * it;
    if (i >= nrow * nch) break;
    const int r = i / nch, c = i - r * nch, q = t0 + r;
    st16(xs + r * kCoPitch + 8 * c, q < CTX ? v[it] : snake8(v[it], a_s + 8 * c, ib_s + 8 * c));
  }
  __syncthreads();
  if (tb == 0) {  // the new state: the last CTX activated rows (this workgroup has read the old state above)
    for (int i = tid; i < CTX * nch; i += 256) {
      const int r = i / nch, c = i - r * nch;
      st16(sb + (int64_t)r * s_st + 8 * c,
           snake8(ld16(xb + (int64_t)(T - CTX + r) * s_xt + 8 * c), a_s + 8 * c, ib_s + 8 * c));
    }
  }
  // Z over the staged rows: wave wv takes 16-row blocks wv, wv + 4, ...; lane (g, r16) supplies row r16 of a
  // block and channels 32 s + 8 g .. + 7 (A), and tap r16's weights for the same channels (B); the C layout
  // leaves Z[4 g + i][tap r16] in lane (g, r16). Channels past Cin and taps past `taps` are zeros.
  const int lane = tid & 63, wv = tid >> 6, r16 = lane & 15, g = lane >> 4;
  const int ksteps = (Cin + 31) >> 5;
  u32x4 bw[kCoMaxCin / 32];
#pragma unroll
  for (int s = 0; s < kCoMaxCin / 32; ++s) {
    const int c = 32 * s + 8 * g;
    bw[s] = (r16 < taps && c < Cin) ? ld16(ws + r16 * Cin + c) : u32x4{0u, 0u, 0u, 0u};
  }
  const int nblk = (nrow + 15) >> 4;
  constexpr int kZP = 9;  // Z row pitch (floats): the final reads of consecutive rows fall on distinct banks
  constexpr int kZBlk = (kCoT + kCoMaxTaps + 15) / 16;
  f32x4 z[(kZBlk + 3) / 4];
#pragma unroll
  for (int q = 0; q < (kZBlk + 3) / 4; ++q) {
    const int blk = wv + 4 * q;
    z[q] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (blk >= nblk) continue;  // (wave-uniform)
    const int r = 16 * blk + r16;
#pragma unroll
    for (int s = 0; s < kCoMaxCin / 32; ++s) {
      if (s >= ksteps) break;
      const int c = 32 * s + 8 * g;
      const u32x4 av = (r < nrow && c < Cin) ? ld16(xs + r * kCoPitch + c) : u32x4{0u, 0u, 0u, 0u};
      z[q] = mfma16x16x32_f16(av, bw[s], z[q]);
    }
  }
  __syncthreads();  // every wave is done with the staged rows: Z goes where they were
  float *zs = reinterpret_cast<float *>(xs);
#pragma unroll
  for (int q = 0; q < (kZBlk + 3) / 4; ++q) {
    const int blk = wv + 4 * q;
    if (blk < nblk && r16 < kCoMaxTaps)
#pragma unroll
      for (int i = 0; i < 4; ++i) zs[(16 * blk + 4 * g + i) * kZP + r16] = z[q][i];
  }
  __syncthreads();
  const int t = t0 + tid;
  if (tid >= kCoT || t >= T) return;
  float acc = 0.f;
  for (int j = 0; j < taps; ++j) acc += zs[(tid + j) * kZP + j];
  acc += bias ? h_lo((uint32_t)bias[0]) : 0.f;
  const float yh = h_lo(pack_f16x2(acc, 0.f));  // the fp16 conv output
  y[(int64_t)b * s_yb + t] = tanhf(yh);
}

static inline bool al16(const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

// The launch shape of one conv: BN = 16 NT output channels and BM = 64 WM rows (NT in 4, 6, 8, 12, 16; WM in
// 1, 2) as conv_plan ranks them (four row tiles per wave measured slower: fewer waves per SIMD); k slices of
// 64 channels when Cin allows, else 96, else 32; when fewer than 512 workgroups remain over a K of >= 16
// slices (the decoder's early, short blocks), K is split into enough shares for ~512 workgroups (at most 6,
// each >= 8 slices; fewer shares measured faster: less workspace to finish),
// summed in fixed order by k_conv_fin from an fp32 workspace.
struct ConvPlan {
  int NT, WM, KSUB, ksplit;
  int64_t ntiles, ws_bytes;
};
// allow_split = false: the caller has no workspace (one pass over K, and the narrow shape that goes with it).
static ConvPlan conv_plan(int64_t M, int Cin, int Cout, int taps, int ph, bool allow_split = true) {
  // 96-channel slices only where K has several of them (a 1x1 conv of 96 channels would be one step with
  // nothing to overlap: measured slower than three 32-channel steps)
  ConvPlan pl{16, 1, Cin % 64 == 0 ? 2 : (Cin % 96 == 0 && taps > 1) ? 3 : 1, 1, 0, 0};
  // (NT, WM) candidates: the fewest padded columns; then, among shapes that fill the chip (>= 512
  // workgroups), the most row tiles per wave (each LDS weight read feeds WM MFMAs), then the widest tile;
  // when none fills it, the most workgroups
  static const int cand[][2] = {{16, 2}, {16, 1}, {12, 2}, {12, 1}, {8, 2}, {8, 1}, {6, 2}, {6, 1}, {4, 2}, {4, 1}};
  int64_t best_cols = INT64_MAX, best_wgs = 0;
  int best_wm = 0;
  for (const auto &c : cand) {
    const int nt = c[0], wm = c[1];
    const int64_t nti = (Cout + 16 * nt - 1) / (16 * nt), cols = nti * 16 * nt;
    const int64_t wgs = ((M + 64 * wm - 1) / (64 * wm)) * nti * ph;
    bool better;
    if (cols != best_cols) better = cols < best_cols;
    else if ((wgs >= 512) != (best_wgs >= 512)) better = wgs >= 512;
    else if (wgs >= 512) better = wm > best_wm;  // candidates come widest first
    else better = wgs > best_wgs;
    if (better) best_cols = cols, best_wgs = wgs, best_wm = wm, pl.NT = nt, pl.WM = wm;
  }
  const int steps = taps * ((Cin + 32 * pl.KSUB - 1) / (32 * pl.KSUB));
  const bool fin_fits = (int64_t)ph * M * ((Cout + 3) / 4) < ((int64_t)1 << 31);
  // multi-tap convs and many-phase transposed convs on short inputs (the decoder's input conv and first
  // block): a wide two-row-tile shape with K split across workgroups beat the narrow tile that fills the
  // chip by itself (block 0's k=7 convs 138 -> 93 us, its stride-8 transposed conv 87 -> 77 us). Only with
  // the split: alone, the wide tile leaves most of the chip idle.
  if ((taps > 2 || ph >= 8) && pl.NT * pl.WM < 16 && best_wgs < 1024 && allow_split && steps >= 16 && fin_fits) {
    for (int nt : {12, 8, 16}) {
      const int64_t nti = (Cout + 16 * nt - 1) / (16 * nt);
      if (nti * 16 * nt != best_cols) continue;
      const int64_t wide_wgs = ((M + 127) / 128) * nti * ph;
      if (wide_wgs >= 512) break;  // K would not be split: keep the narrow tile
      pl.NT = nt;
      pl.WM = 2;
      best_wgs = wide_wgs;
      break;
    }
  }
  // shapes that would not fit two workgroups per CU: 96-channel slices of 12 / 16 column tiles (> 80 KB of
  // LDS) take 32-channel slices; two row tiles of 16 column tiles (> 256 registers) take one
  if (pl.KSUB == 3 && pl.NT >= 12) pl.KSUB = 1;
  if (pl.WM == 2 && pl.NT == 16 && pl.KSUB >= 2) {
    pl.WM = 1;
    best_wgs = ((M + 63) / 64) * ((Cout + 255) / 256) * ph;
  }
  pl.ntiles = (Cout + 16 * pl.NT - 1) / (16 * pl.NT);
  const int64_t wgs = best_wgs;
  if (allow_split && wgs < 512 && steps >= 16 && fin_fits) {
    int64_t k = (512 + wgs - 1) / wgs;
    k = k < steps / 8 ? k : steps / 8;
    k = k < 6 ? k : 6;  // more shares measured slower (the input conv: 11 shares 58 us, 6 shares 51 us)
    if (k > 1) {
      pl.ksplit = (int)k;
      pl.ws_bytes = k * ph * M * pl.ntiles * 16 * pl.NT * 4;
    }
  }
  return pl;
}

}  // namespace a8

extern "C" int a8_conv_cl(const void *x, int64_t s_xb, int64_t s_xt, const void *w, int64_t s_wp, int64_t s_wt,
                          int64_t s_wc, int cout_w, const void *bias, const void *res, int64_t s_rb, int64_t s_rt,
                          void *y, int64_t s_yb, int64_t s_yt, const float *snake_a, const float *snake_ib, int B,
                          int Tin, int TR, int Cin, int Cout, int taps, int dil, int ph, void *ws, int64_t ws_bytes,
                          void *stream) {
  using namespace a8;
  if (B < 0 || TR < 0 || Cin <= 0 || Cout <= 0 || taps <= 0 || dil <= 0 || ph <= 0 || cout_w < Cout)
    return set_error(A8_EINVAL, "conv_cl: bad sizes B=%d TR=%d Cin=%d Cout=%d taps=%d dil=%d ph=%d cout_w=%d", B, TR,
                     Cin, Cout, taps, dil, ph, cout_w);
  if ((int64_t)TR + (int64_t)(taps - 1) * dil > Tin)
    return set_error(A8_EINVAL, "conv_cl: %d input rows, %d needed", Tin, TR + (taps - 1) * dil);
  if (Cin % 8) return set_error(A8_EUNSUP, "conv_cl: Cin %d not a multiple of 8", Cin);
  if (snake_a && Cin > kSnakeMaxC)
    return set_error(A8_EUNSUP, "conv_cl: the snake on the load takes Cin <= %d (got %d; use snake_cat)", kSnakeMaxC, Cin);
  if (B == 0 || TR == 0) return 0;
  if (!x || !w || !y || (snake_a != nullptr) != (snake_ib != nullptr))
    return set_error(A8_EINVAL, "conv_cl: null pointer");
  // y (and res) may be any 2-byte-aligned view: the epilogue stores element by element unless 8-byte stores of
  // four channels are aligned. The weight rows are read 16 bytes at a time: cout_w (its padded width) must be a
  // multiple of 8.
  if (!al16(x) || !al16(w) || (s_xb | s_xt | s_wp | s_wt | s_wc) & 7 || (cout_w & 7) ||
      (snake_a && (!al16(snake_a) || !al16(snake_ib))) || (reinterpret_cast<uintptr_t>(y) & 1u) ||
      (res && (reinterpret_cast<uintptr_t>(res) & 1u)))
    return set_error(A8_EALIGN, "conv_cl: x / w / snake 16-byte aligned, their strides and the weight's padded "
                     "width (%d) multiples of 8", cout_w);
  const int64_t M = (int64_t)B * TR;
  if (M > INT32_MAX / 2) return set_error(A8_EUNSUP, "conv_cl: %lld rows too many", (long long)M);
  // bytes the kernel may read from x and w: both are addressed by 32-bit buffer offsets
  const int64_t x_span = ((int64_t)(B - 1) * s_xb + (int64_t)(Tin - 1) * s_xt + Cin) * 2;
  const int64_t w_span = ((int64_t)(ph - 1) * s_wp + (int64_t)(taps - 1) * s_wt + (int64_t)(Cin - 1) * s_wc + cout_w) * 2;
  if (x_span >= ((int64_t)1 << 31) || w_span >= ((int64_t)1 << 31) || s_xb < 0 || s_xt < 0 || s_wp < 0 || s_wt < 0 ||
      s_wc < 0)
    return set_error(A8_EUNSUP, "conv_cl: x spans %lld bytes, w %lld (each must be below 2 GiB, strides >= 0)",
                     (long long)x_span, (long long)w_span);
  ConvPlan pl = conv_plan(M, Cin, Cout, taps, ph);
  if (pl.ksplit > 1 && (!ws || ws_bytes < pl.ws_bytes)) pl = conv_plan(M, Cin, Cout, taps, ph, false);  // one pass
  if (pl.ksplit > 1 && !al16(ws)) return set_error(A8_EALIGN, "conv_cl: workspace must be 16-byte aligned");
  const int NT = pl.NT, WM = pl.WM;
  float *part = pl.ksplit > 1 ? (float *)ws : nullptr;
  const dim3 grid((unsigned)((M + 64 * WM - 1) / (64 * WM)), (unsigned)pl.ntiles, (unsigned)(ph * pl.ksplit));
#define A8_CONV_ARGS (const uint16_t *)x, s_xb, s_xt, (const uint16_t *)w, s_wp, s_wt, s_wc, (const uint16_t *)bias, \
                     (const uint16_t *)res, s_rb, s_rt, (uint16_t *)y, s_yb, s_yt, snake_a, snake_ib, (int)M, TR, Cin, \
                     Cout, cout_w, taps, dil, ph, part, pl.ksplit, (uint32_t)x_span, (uint32_t)w_span, nullptr,     \
                     nullptr, nullptr, nullptr, 0u
#define A8_CONV_L(wm, nt, ksub, sn) \
  hipLaunchKernelGGL((k_conv_cl<wm, nt, ksub, sn>), grid, dim3(256), 0, (hipStream_t)stream, A8_CONV_ARGS)
#define A8_CONV_NT(wm, ksub, sn)                 \
  switch (NT) {                                  \
    case 4: A8_CONV_L(wm, 4, ksub, sn); break;   \
    case 6: A8_CONV_L(wm, 6, ksub, sn); break;   \
    case 8: A8_CONV_L(wm, 8, ksub, sn); break;   \
    case 12: A8_CONV_L(wm, 12, ksub, sn); break; \
    default: A8_CONV_L(wm, 16, ksub, sn); break; \
  }
#define A8_CONV_NT_NARROW(wm, ksub, sn)        \
  switch (NT) {                                \
    case 4: A8_CONV_L(wm, 4, ksub, sn); break; \
    case 6: A8_CONV_L(wm, 6, ksub, sn); break; \
    default: A8_CONV_L(wm, 8, ksub, sn); break; \
  }
#define A8_CONV_NT_NO16(wm, ksub, sn)            \
  switch (NT) {                                  \
    case 4: A8_CONV_L(wm, 4, ksub, sn); break;   \
    case 6: A8_CONV_L(wm, 6, ksub, sn); break;   \
    case 8: A8_CONV_L(wm, 8, ksub, sn); break;   \
    default: A8_CONV_L(wm, 12, ksub, sn); break; \
  }
  // (conv_plan keeps KSUB 3 to NT <= 8 and two row tiles with KSUB 2 to NT <= 12: those instances are the
  // ones that fit two workgroups per CU)
#define A8_CONV_K(wm, sn)              \
  if (pl.KSUB == 2) {                  \
    if (wm == 2) {                     \
      A8_CONV_NT_NO16(2, 2, sn)        \
    } else {                           \
      A8_CONV_NT(1, 2, sn)             \
    }                                  \
  } else if (pl.KSUB == 3) {           \
    A8_CONV_NT_NARROW(wm, 3, sn)       \
  } else {                             \
    A8_CONV_NT(wm, 1, sn)              \
  }
  if (WM == 2) {
    if (snake_a) {
      A8_CONV_K(2, true)
    } else {
      A8_CONV_K(2, false)
    }
  } else {
    if (snake_a) {
      A8_CONV_K(1, true)
    } else {
      A8_CONV_K(1, false)
    }
  }
#undef A8_CONV_K
#undef A8_CONV_L
#undef A8_CONV_NT
#undef A8_CONV_NT_NARROW
#undef A8_CONV_NT_NO16
#undef A8_CONV_ARGS
  if (part) {
    const hipError_t e = hipGetLastError();  // the finish would sum a workspace the main launch never wrote
    if (e != hipSuccess) return (int)e;
    const int64_t threads = (int64_t)ph * M * ((Cout + 3) / 4);
    hipLaunchKernelGGL(k_conv_fin, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const float *)part, pl.ntiles * 16 * NT, pl.ksplit, (const uint16_t *)bias,
                       (const uint16_t *)res, s_rb, s_rt, (uint16_t *)y, s_yb, s_yt, (int)M, TR, Cout, ph);
  }
  return (int)hipGetLastError();
}

extern "C" int64_t a8_conv_cl_ws_bytes(int B, int TR, int Cin, int Cout, int taps, int ph) {
  using namespace a8;
  if (B <= 0 || TR <= 0 || Cin <= 0 || Cout <= 0 || taps <= 0 || ph <= 0) return 0;
  const int64_t M = (int64_t)B * TR;
  if (M > INT32_MAX / 2) return 0;
  return conv_plan(M, Cin, Cout, taps, ph).ws_bytes;
}

extern "C" int a8_ru_cl(const void *xin, int64_t s_xb, int64_t s_xt, const void *w1, int64_t s_wt, int64_t s_wc,
                        const void *b1, const float *a2, const float *ib2, const void *w2, const void *b2,
                        const void *res, int64_t s_rb, int64_t s_rt, void *y, int64_t s_yb, int64_t s_yt, int B,
                        int Tin, int TR, int C, int taps, int dil, void *stream) {
  using namespace a8;
  if (B < 0 || TR < 0 || C <= 0 || taps <= 0 || dil <= 0)
    return set_error(A8_EINVAL, "ru_cl: bad sizes B=%d TR=%d C=%d taps=%d dil=%d", B, TR, C, taps, dil);
  if ((int64_t)TR + (int64_t)(taps - 1) * dil > Tin)
    return set_error(A8_EINVAL, "ru_cl: %d input rows, %d needed", Tin, TR + (taps - 1) * dil);
  if (C != 96 && C != 192 && C != 384)
    return set_error(A8_EUNSUP, "ru_cl: %d channels (96, 192 or 384: one tile holds the row)", C);
  if (B == 0 || TR == 0) return 0;
  if (!xin || !w1 || !b1 || !a2 || !ib2 || !w2 || !b2 || !res || !y) return set_error(A8_EINVAL, "ru_cl: null pointer");
  if (!al16(xin) || !al16(w1) || !al16(w2) || !al16(a2) || !al16(ib2) || (reinterpret_cast<uintptr_t>(b1) & 7u) ||
      (s_xb | s_xt | s_wt) & 7 || s_wc != C || (reinterpret_cast<uintptr_t>(y) & 1u) ||
      (reinterpret_cast<uintptr_t>(res) & 1u))
    return set_error(A8_EALIGN, "ru_cl: xin / w1 / w2 / a2 / ib2 16-byte aligned, b1 8, strides multiples of 8, "
                     "weight rows of C = %d", C);
  const int64_t M = (int64_t)B * TR;
  if (M > INT32_MAX / 2) return set_error(A8_EUNSUP, "ru_cl: %lld rows too many", (long long)M);
  const int64_t x_span = ((int64_t)(B - 1) * s_xb + (int64_t)(Tin - 1) * s_xt + C) * 2;
  const int64_t w_span = ((int64_t)(taps - 1) * s_wt + (int64_t)(C - 1) * s_wc + C) * 2;
  const int64_t w2_span = ((int64_t)(C - 1) * s_wc + C) * 2;
  if (x_span >= ((int64_t)1 << 31) || w_span >= ((int64_t)1 << 31) || s_xb < 0 || s_xt < 0 || s_wt < 0)
    return set_error(A8_EUNSUP, "ru_cl: xin spans %lld bytes, w1 %lld (each must be below 2 GiB)", (long long)x_span,
                     (long long)w_span);
  // the whole row in one tile (NT = C / 16); two row tiles per wave where that still gives >= 512 workgroups
  // (384 channels: one row tile and 32-channel slices, to stay within two workgroups per CU)
  const int WM = C <= 192 && (M + 127) / 128 >= 512 ? 2 : 1;
  const dim3 grid((unsigned)((M + 64 * WM - 1) / (64 * WM)), 1u, 1u);
#define A8_RU_L(wm, nt, ksub)                                                                                        \
  hipLaunchKernelGGL((k_conv_cl<wm, nt, ksub, false, true>), grid, dim3(256), 0, (hipStream_t)stream,                \
                     (const uint16_t *)xin, s_xb, s_xt, (const uint16_t *)w1, (int64_t)0, s_wt, s_wc,                \
                     (const uint16_t *)b1, (const uint16_t *)res, s_rb, s_rt, (uint16_t *)y, s_yb, s_yt, nullptr,     \
                     nullptr, (int)M, TR, C, C, C, taps, dil, 1, nullptr, 1, (uint32_t)x_span, (uint32_t)w_span,     \
                     (const uint16_t *)w2, (const uint16_t *)b2, a2, ib2, (uint32_t)w2_span)
  if (C == 384) {
    A8_RU_L(1, 24, 1);
  } else if (C == 192) {
    if (WM == 2) A8_RU_L(2, 12, 2); else A8_RU_L(1, 12, 2);
  } else {
    if (WM == 2) A8_RU_L(2, 6, 3); else A8_RU_L(1, 6, 3);
  }
#undef A8_RU_L
  return (int)hipGetLastError();
}

static int snake_cat_entry(const char *fn, const void *x, int64_t s_xb, int64_t s_xt, const void *state, int64_t s_sb,
                           int64_t s_st, const float *a, const float *ib, void *y, int64_t s_yb, int64_t s_yt, int B,
                           int T, int CTX, int C, bool refresh, void *stream) {
  using namespace a8;
  if (B < 0 || T < 0 || CTX < 0 || C <= 0) return set_error(A8_EINVAL, "%s: bad sizes B=%d T=%d CTX=%d C=%d", fn, B, T, CTX, C);
  if (C % 8) return set_error(A8_EUNSUP, "%s: C %d not a multiple of 8", fn, C);
  if (refresh && T < CTX)
    return set_error(A8_EUNSUP, "%s: the state refresh needs T >= CTX (T %d, CTX %d)", fn, T, CTX);
  if (B == 0 || T + CTX == 0) return 0;
  if ((T > 0 && !x) || (CTX > 0 && !state) || !y || (a != nullptr) != (ib != nullptr))
    return set_error(A8_EINVAL, "%s: null pointer", fn);
  if ((x && !al16(x)) || (state && !al16(state)) || !al16(y) || (a && (!al16(a) || !al16(ib))) ||
      (s_xb | s_xt | s_sb | s_st | s_yb | s_yt) & 7)
    return set_error(A8_EALIGN, "%s: pointers 16-byte aligned, strides multiples of 8", fn);
  const int64_t n = (int64_t)B * (refresh ? T : CTX + T) * (C / 8);
  if (n >= (int64_t)1 << 31) return set_error(A8_EUNSUP, "%s: too large", fn);
  const unsigned grid = (unsigned)((n + 255) / 256);
  auto kern = a ? (refresh ? k_snake_cat<true, true> : k_snake_cat<true, false>)
                : (refresh ? k_snake_cat<false, true> : k_snake_cat<false, false>);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const uint16_t *)x, s_xb, s_xt,
                     (uint16_t *)const_cast<void *>(state), s_sb, s_st, a, ib, (uint16_t *)y, s_yb, s_yt, B, T, CTX, C);
  return (int)hipGetLastError();
}

extern "C" int a8_snake_cat(const void *x, int64_t s_xb, int64_t s_xt, const void *state, int64_t s_sb, int64_t s_st,
                            const float *a, const float *ib, void *y, int64_t s_yb, int64_t s_yt, int B, int T, int CTX,
                            int C, void *stream) {
  return snake_cat_entry("snake_cat", x, s_xb, s_xt, state, s_sb, s_st, a, ib, y, s_yb, s_yt, B, T, CTX, C, false,
                         stream);
}

extern "C" int a8_snake_cat_refresh(const void *x, int64_t s_xb, int64_t s_xt, void *state, int64_t s_sb, int64_t s_st,
                                    const float *a, const float *ib, void *y, int64_t s_yb, int64_t s_yt, int B, int T,
                                    int CTX, int C, void *stream) {
  return snake_cat_entry("snake_cat_refresh", x, s_xb, s_xt, state, s_sb, s_st, a, ib, y, s_yb, s_yt, B, T, CTX, C,
                         true, stream);
}

extern "C" int a8_conv_out_tanh(const void *x, int64_t s_xb, int64_t s_xt, void *state, int64_t s_sb, int64_t s_st,
                                const float *a, const float *ib, const void *w, const void *bias, float *y, int64_t s_yb,
                                int B, int T, int CTX, int Cin, int taps, void *stream) {
  using namespace a8;
  if (B < 0 || T < 0 || CTX < 0 || Cin <= 0 || taps <= 0)
    return set_error(A8_EINVAL, "conv_out_tanh: bad sizes B=%d T=%d CTX=%d Cin=%d taps=%d", B, T, CTX, Cin, taps);
  if (Cin % 8 || Cin > kCoMaxCin || taps > kCoMaxTaps || CTX != taps - 1 || T < CTX)
    return set_error(A8_EUNSUP, "conv_out_tanh: Cin %d (a multiple of 8 up to %d), taps %d (up to %d), context %d (taps - 1), "
                     "T %d >= context", Cin, kCoMaxCin, taps, kCoMaxTaps, CTX, T);
  if (B == 0 || T == 0) return 0;
  if (!x || (CTX > 0 && !state) || !a || !ib || !w || !y) return set_error(A8_EINVAL, "conv_out_tanh: null pointer");
  if (!al16(x) || (state && !al16(state)) || !al16(a) || !al16(ib) || !al16(w) || (s_xb | s_xt | s_sb | s_st) & 7)
    return set_error(A8_EALIGN, "conv_out_tanh: pointers 16-byte aligned, strides multiples of 8");
  const int64_t grid = (int64_t)B * ((T + kCoT - 1) / kCoT);
  if (grid >= (int64_t)1 << 31) return set_error(A8_EUNSUP, "conv_out_tanh: too large");
  hipLaunchKernelGGL(k_conv_out, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, (const uint16_t *)x, s_xb, s_xt,
                     (uint16_t *)state, s_sb, s_st, a, ib, (const uint16_t *)w, (const uint16_t *)bias, y, s_yb, T, CTX,
                     Cin, taps);
  return (int)hipGetLastError();
}
