// Small-M GEMM for the slow-AR layer's projections (a8_gemm_small): out[M, N] = bf16(X[M, K] . W[N, K]^T), fp32
// accumulation, for the decode tick's token counts (M <= 192: the 192 slots of C3). It takes the place of the
// reference's per-shape GEMM choice for small M (serve/fast_kernels.py:413-519, GemmDispatch: cuBLAS or a tuned
// Triton config; here hipBLASLt or this kernel, chosen per (M, N, K) by timing, as there).
//
// What bounds it at these shapes: the weights (2-17 MB per projection) stream from HBM once, and every workgroup
// re-reads the token rows X (344 KB at K = 896) from L2, at ~60 bytes per clock per CU (measured) -- so the
// workgroup tile is all M rows x 64 weight rows, and K is split across workgroups only for narrow N.
//
// One workgroup = 64 weight rows (four 16-row n-subtiles) x all token rows (MT 16-row m-subtiles, MT even)
// x a range of KC-wide k chunks (KC = 128 for token tiles of up to 64 rows where K allows, else 64: each wait
// and meeting then covers twice the bytes, measured 0.2-1.3 us faster per product at the slow AR's shapes). The
// chunk's X rows and W rows go from HBM / L2 into LDS by DMA (16-byte pieces, row r's KC / 8 pieces permuted by
// piece ^= r mod KC / 8 through the source offsets so the operand reads of consecutive rows spread over the
// banks): the weights through a ring of 8 slots with 7 chunks in flight at KC = 64 (5 and 4 at KC = 128, the
// same bytes; they come from HBM: ~1.5 us away), the token rows through a ring of 3 with 2 in flight (L2).
// Wave w computes n-subtiles 2(w&1), 2(w&1)+1 x m-subtiles (w>>1) MT/2.. : per 32-k step two W operands and
// MT/2 X operands from LDS, MT MFMAs (v_mfma_f32_16x16x32_bf16: A = W rows, B = X^T, so the C layout holds 4 consecutive output
// columns of one token row per lane). The DMA is inline asm the compiler does not track; the kernel waits for
// it with vmcnt counts (every wave issues the same number of requests per chunk, and loads complete in order).
// The token rows may also be split into row blocks (blockIdx.z), for more workgroups where N is narrow. With
// several k splits each workgroup writes fp32 partials (sc1 stores, coherent across the XCDs) and the tile's
// last workgroup to arrive, known from a counter at the start of the workspace, sums them in a fixed order in
// the same launch (no device-scope fence: that would write back and invalidate the whole XCD L2 under the
// other workgroups' loads, measured 5-20x slower than the GEMM).
#include <algorithm>
#include <type_traits>

#include "a8_common.h"

namespace a8 {
namespace {

constexpr int kGmNB = 64;   // weight rows per workgroup
constexpr int kGmKC = 64;   // k granularity (the narrower chunk; K must be a multiple of it)
constexpr int kGmWSlots = 8;  // W ring slots at 64-wide chunks: 7 chunks of weights in flight (HBM latency), X 2 (L2)
constexpr int kGmMaxM = 192;
constexpr int kGmCntBytes = 4096;  // k splits: the workspace starts with one 32-bit counter per tile (<= 1024)
constexpr int kGmSsMax = 32;       // norm-fused products: partial sums of squares per row (N / 32 <= 32)

__device__ __forceinline__ void gm_dma(u32x4 rs, uint32_t lds, uint32_t voff) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" : : "{m0}"(lds), "v"(voff), "s"(rs) : "memory");
}
__device__ __forceinline__ u32x4 gm_rsrc(const void *base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xFFFFu, bytes, 0x00020000u};
}
template <int N>
__device__ __forceinline__ void gm_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Epilogue options of the norm-fused projections (a8_gemm_small_norm; zero / null: the plain product):
//   res_add  out is the residual stream: out = bf16(f32(bf16(acc)) + f32(out)) in place (the reference's
//            o / w2 product rounded to bf16, then rmsnorm's residual add, fast_kernels.py:30-46);
//   ss_out   with res_add: per token row and 32-column group, the sum of squares of the new residual values
//            (fp32 [Mall][N / 32]: the next RMSNorm's statistic, summed by its consumer);
//   ss_in    the token rows are a raw residual stream h whose RMSNorm (weight folded into w by the caller) this
//            product consumes: acc is scaled by rsqrt(sum_j ss_in[m][j] / K + eps) before the rounding.
//   pf       workgroups z >= pf_z0 of the grid only read [pf, pf + pf_n16 16-byte pieces) once and end: the next
//            product's weights into the memory-side cache while this product's own workgroups (fewer than the
//            chip's compute units) leave the bandwidth idle; pf_sink takes a word in a case that never happens.
struct GmEpi {
  int res_add;
  float *ss_out;
  const float *ss_in;
  int ss_n;
  float eps;
  const u32x4 *pf;
  int64_t pf_n16;
  uint32_t *pf_sink;
  int pf_z0;
};

template <int MT, int NW, int KC>
__global__ __launch_bounds__(64 * NW, 1) void k_gemm_small(const uint16_t *__restrict__ x, int64_t ldx,
                                                           const uint16_t *__restrict__ w, int64_t ldw,
                                                           uint16_t *__restrict__ out, int64_t ldo,
                                                           float *__restrict__ part, int32_t *__restrict__ cnt,
                                                           int Mall, int N, int K, int cps, int S, int I, GmEpi ep) {
  static_assert(NW == 4 || NW == 8, "waves");
  static_assert(MT >= 2 && MT * 16 <= kGmMaxM && (2 * MT) % NW == 0, "token subtiles");
  warm_kernargs<152>();  // the explicit arguments above span 0x00-0x97
  if (ep.pf && (int)blockIdx.z >= ep.pf_z0) {  // a prefetch workgroup (uniform: no barrier below is reached)
    const int64_t tpw = 64 * NW;
    const int64_t id = ((int64_t)(blockIdx.z - ep.pf_z0) * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    const int64_t stride = (int64_t)gridDim.x * gridDim.y * (gridDim.z - ep.pf_z0) * tpw;
    uint32_t acc = 0;
    for (int64_t i = id * tpw + threadIdx.x; i < ep.pf_n16; i += 8 * stride) {
      u32x4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = i + u * stride < ep.pf_n16 ? ep.pf[i + u * stride] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int u = 0; u < 8; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    if (acc == 0x9E3779B9u) ep.pf_sink[threadIdx.x & 3] = acc;
    return;
  }
  static_assert(KC == 64 || KC == 128, "k chunk");
  constexpr int CPR = KC / 8;              // 16-byte pieces of a row's chunk
  constexpr int RB = 2 * KC;               // bytes of a row's chunk
  constexpr int RPI = 64 / CPR;            // rows per 1 KB request
  constexpr int XB = MT * 16 * RB;         // X bytes per ring slot
  constexpr int WB = kGmNB * RB;           // W bytes per ring slot
  constexpr int DX = MT * 16 / RPI / NW;   // X requests per wave per chunk
  constexpr int DW = kGmNB / RPI / NW;     // W requests per wave per chunk
  constexpr int KS = KC / 32;              // 32-k MFMA steps per chunk
  constexpr int WSL = KC == 64 ? kGmWSlots : 5;  // W ring slots (the same bytes in flight)
  constexpr int MH = 2 * MT / NW;          // m-subtiles per wave (waves: 2 along n x NW / 2 along m)
  static_assert(DX * NW * RPI == MT * 16 && DW * NW * RPI == kGmNB, "requests");
  __shared__ __attribute__((aligned(16))) char lds[3 * XB + WSL * WB];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int r16 = lane & 15, g = lane >> 4;
  const int nt = blockIdx.x, sp = blockIdx.y;
  // row block z: token rows z MT 16 .. of the Mall rows (the host picks MT so that the blocks cover them)
  const int mb0 = (int)blockIdx.z * MT * 16, M = min(MT * 16, Mall - mb0);
  x += (int64_t)mb0 * ldx;
  out += (int64_t)mb0 * ldo;
  const int nch = K / KC;
  const int c0 = sp * cps, c1 = min(c0 + cps, nch);
  if (c0 >= c1) return;  // (the host sizes the grid so that this does not happen)
  const int n0 = nt * kGmNB;

  // sources: rows past M / N read as zeros (their offsets lie past the range: ld >= K); a chunk past the
  // workgroup's range is requested from an empty range (zeros into a free slot, no memory traffic), so every
  // wave issues the same requests every chunk and the waits below are constant
  // gated (I > 0: w = [gate; up], I rows each, out = silu(x gate^T) * (x up^T), I columns): the tile's weight
  // rows 0..31 are gate rows 32 nt.., rows 32..63 the up rows I + 32 nt.. -- 32 output columns a workgroup
  const bool gated = I > 0;
  const int wrow0 = gated ? 32 * nt : n0, wlim = gated ? I : N;
  const uint32_t wbytes = (uint32_t)((int64_t)(wlim - wrow0 - 1) * ldw * 2 + (int64_t)K * 2);
  const u32x4 xr = gm_rsrc(x, (uint32_t)((int64_t)(M - 1) * ldx * 2 + (int64_t)K * 2));
  const u32x4 wr = gm_rsrc(w + (int64_t)wrow0 * ldw, wbytes);
  const u32x4 wu = gated ? gm_rsrc(w + (int64_t)(I + wrow0) * ldw, wbytes) : wr;
  u32x4 xr0 = xr, wr0 = wr;
  xr0[2] = 0u;
  wr0[2] = 0u;
  const uint32_t prow = (uint32_t)lane / (uint32_t)CPR, pch = (uint32_t)lane % (uint32_t)CPR;
  uint32_t xso[DX], xdo[DX], wso[DW], wdo[DW];
  u32x4 wres[DW];
#pragma unroll
  for (int j = 0; j < DX; ++j) {  // X instruction i = wv + NW j: token rows 8i..8i+7
    const uint32_t i = (uint32_t)(wv + NW * j), row = (uint32_t)RPI * i + prow;
    xso[j] = row * (uint32_t)(ldx * 2) + ((pch ^ (row & (uint32_t)(CPR - 1))) << 4);
    xdo[j] = i * 1024u;
  }
#pragma unroll
  for (int j = 0; j < DW; ++j) {  // W instruction i = wv + NW j: weight rows 8i..8i+7 of the tile
    const uint32_t i = (uint32_t)(wv + NW * j), row = (uint32_t)RPI * i + prow;
    const bool up = gated && i >= (uint32_t)(32 / RPI);  // (wave-uniform) the up half of a gated tile, from its own source
    wres[j] = up ? wu : wr;
    const uint32_t srow = up ? row - 32u : row;
    wso[j] = srow * (uint32_t)(ldw * 2) + ((pch ^ (row & (uint32_t)(CPR - 1))) << 4);
    wdo[j] = i * 1024u;
  }
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(lds);
  const uint32_t wring = lds0 + 3u * XB;
  auto issue_x = [&](int c, int slot) __attribute__((always_inline)) {
    const u32x4 rs = c < c1 ? xr : xr0;
    const uint32_t kb = (uint32_t)(c * KC * 2);
#pragma unroll
    for (int j = 0; j < DX; ++j) gm_dma(rs, lds0 + (uint32_t)(slot * XB) + xdo[j], xso[j] + kb);
  };
  auto issue_w = [&](int c) __attribute__((always_inline)) {
    const uint32_t kb = (uint32_t)(c * KC * 2);
    const uint32_t slot = (uint32_t)(c - c0) % (uint32_t)WSL;
#pragma unroll
    for (int j = 0; j < DW; ++j) gm_dma(c < c1 ? wres[j] : wr0, wring + slot * WB + wdo[j], wso[j] + kb);
  };

  // operand reads: lane (g, r16) takes row r16 of a subtile, k 8g..8g+7 of the 32-k step s (chunk 4s + g)
  const int jn0 = 2 * (wv & 1), im0 = (wv >> 1) * MH;
  f32x4 acc[2][MH];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < MH; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ss_in: thread m < M loads row m's partial sums of squares now, ahead of every DMA request (loads complete in
  // order, so the first chunk's wait covers them), and parks 1 / rms in LDS after that wait
  __shared__ float inv_s[kGmMaxM];
  f32x4 ssv[kGmSsMax / 4];
  const bool has_ss = ep.ss_in != nullptr;
  if (has_ss && (int)threadIdx.x < M) {
    const float *sp4 = ep.ss_in + (int64_t)(mb0 + (int)threadIdx.x) * ep.ss_n;
#pragma unroll
    for (int j = 0; j < kGmSsMax / 4; ++j)
      ssv[j] = 4 * j < ep.ss_n ? *reinterpret_cast<const f32x4 *>(sp4 + 4 * j) : f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // res_add without k splits: this lane's old residual values, requested ahead of the DMA as well
  u32x2 rold[2][MH];
  if (ep.res_add && !part) {
#pragma unroll
    for (int b = 0; b < MH; ++b)
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int m = 16 * (im0 + b) + r16, n = n0 + 16 * (jn0 + a) + 4 * g;
        rold[a][b] = (m < M && n < N) ? *reinterpret_cast<const u32x2 *>(out + (int64_t)m * ldo + n) : u32x2{0u, 0u};
      }
  }

  // W chunks c0 .. c0 + P - 1 (P = kGmWSlots - 1 in flight), then X chunks c0, c0 + 1; per chunk c: the wait,
  // the meeting (everyone is done with chunk c - 1, whose slots the next requests refill), X(c + 2), W(c + P)
  constexpr int P = WSL - 1;
#pragma unroll
  for (int c = 0; c < P; ++c) issue_w(c0 + c);
  issue_x(c0, 0);
  issue_x(c0 + 1, 1);
  int xs = 0;
  for (int c = c0; c < c1; ++c) {
    // X(c) in LDS (and W(c), requested earlier): at most the requests issued after X(c) outstanding
    if (c == c0)
      gm_wait_vm<DX>();
    else if (c == c0 + 1)
      gm_wait_vm<DX + DW>();
    else
      gm_wait_vm<DX + 2 * DW>();
    lds_barrier();
    issue_x(c + 2, xs == 0 ? 2 : xs - 1);
    issue_w(c + P);
    const char *sx = lds + xs * XB;
    const char *sw = lds + 3 * XB + ((c - c0) % WSL) * WB;
    // every operand of the chunk is read before its first product: one LDS round trip per chunk, not one per
    // pair of products (the scheduler otherwise places each read just before its use)
    u32x4 A[KS][2], B[KS][MH];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint32_t ch = (uint32_t)(4 * s + g);
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const uint32_t row = (uint32_t)(16 * (jn0 + a) + r16);
        A[s][a] = ld16(sw + row * (uint32_t)RB + ((ch ^ (row & (uint32_t)(CPR - 1))) << 4));
      }
#pragma unroll
      for (int b = 0; b < MH; ++b) {
        const uint32_t row = (uint32_t)(16 * (im0 + b) + r16);
        B[s][b] = ld16(sx + row * (uint32_t)RB + ((ch ^ (row & (uint32_t)(CPR - 1))) << 4));
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int b = 0; b < MH; ++b)
#pragma unroll
        for (int a = 0; a < 2; ++a) acc[a][b] = mfma16x16x32(A[s][a], B[s][b], acc[a][b]);
    xs = xs == 2 ? 0 : xs + 1;
  }
  // the requests past the range still write (zeros) into LDS: let them land before the workgroup ends
  gm_wait_vm<0>();
  if (has_ss) {  // 1 / rms of every token row, for the epilogues (the loads above have long returned)
    if ((int)threadIdx.x < M) {
      float t = 0.f;
#pragma unroll
      for (int j = 0; j < kGmSsMax / 4; ++j)  // in order 0 .. ss_n - 1 (the rest are zeros)
        t = (((t + ssv[j][0]) + ssv[j][1]) + ssv[j][2]) + ssv[j][3];
      inv_s[threadIdx.x] = __builtin_amdgcn_rsqf(t / (float)K + ep.eps);
    }
    __syncthreads();
  }

  // lane (g, r16) of tile (a, b): token row 16(im0 + b) + r16, output columns n0 + 16(jn0 + a) + 4g..+3
  if (gated) {
    // a gate wave (even: tile rows 0..31) and the up wave beside it (odd: rows 32..63, same token rows) hold the
    // two halves of the same output columns; each finishes one of its two 16-column subtiles -- the gate wave
    // a = 0, the up wave a = 1 -- taking the other half's values (rounded to bf16, as the GEMM's output would
    // be) from its partner through LDS where the rings were: silu(gate) * up, rounded again
    __syncthreads();  // every wave is done with the rings
    uint32_t *park = reinterpret_cast<uint32_t *>(lds) + (wv >> 1) * (2 * MH * 128);
    if (has_ss) {  // the consumed RMSNorm's 1 / rms, on the fp32 products of both halves
#pragma unroll
      for (int b = 0; b < MH; ++b) {
        const float iv = inv_s[min(16 * (im0 + b) + r16, M - 1)];
#pragma unroll
        for (int a = 0; a < 2; ++a) acc[a][b] *= iv;
      }
    }
    // (acc indexed by constants only: a subtile picked at run time makes the compiler keep acc in LDS, its
    // stores then run inside the k loop)
    auto park_half = [&](auto ap_tag) __attribute__((always_inline)) {
      constexpr int ap = decltype(ap_tag)::value;  // the subtile handed to the partner: slot (ap, b)
#pragma unroll
      for (int b = 0; b < MH; ++b)
        *reinterpret_cast<u32x2 *>(park + (ap * MH + b) * 128 + 2 * lane) =
            u32x2{pack_bf16x2(acc[ap][b][0], acc[ap][b][1]), pack_bf16x2(acc[ap][b][2], acc[ap][b][3])};
    };
    auto finish_half = [&](auto a_tag) __attribute__((always_inline)) {
      constexpr int a = decltype(a_tag)::value;  // the subtile this wave finishes (its partner parked slot (a, b))
      const int n = 32 * nt + 16 * a + 4 * g;
#pragma unroll
      for (int b = 0; b < MH; ++b) {
        const int m = 16 * (im0 + b) + r16;
        if (m >= M || n >= I) continue;
        const u32x2 mine{pack_bf16x2(acc[a][b][0], acc[a][b][1]), pack_bf16x2(acc[a][b][2], acc[a][b][3])};
        const u32x2 other = *reinterpret_cast<const u32x2 *>(park + (a * MH + b) * 128 + 2 * lane);
        const u32x2 gt = a == 0 ? mine : other, up = a == 0 ? other : mine;
        st8(out + (int64_t)m * ldo + n, u32x2{silu_mul_bf16x2(gt[0], up[0]), silu_mul_bf16x2(gt[1], up[1])});
      }
    };
    const bool upw = wv & 1;  // wave-uniform
    if (upw)
      park_half(std::integral_constant<int, 0>{});
    else
      park_half(std::integral_constant<int, 1>{});
    __syncthreads();
    if (upw)
      finish_half(std::integral_constant<int, 1>{});
    else
      finish_half(std::integral_constant<int, 0>{});
    return;
  }
  if (!part) {
#pragma unroll
    for (int b = 0; b < MH; ++b) {
      const int m = 16 * (im0 + b) + r16;
      const float iv = has_ss ? inv_s[min(m, M - 1)] : 1.f;
      float ss = 0.f;
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int n = n0 + 16 * (jn0 + a) + 4 * g;
        u32x2 o{pack_bf16x2(acc[a][b][0] * iv, acc[a][b][1] * iv), pack_bf16x2(acc[a][b][2] * iv, acc[a][b][3] * iv)};
        if (ep.res_add) {  // h = bf16(a + res), a the product rounded to bf16 (zeros outside the tile's range)
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            o[e] = pack_bf16x2(bf_lo(o[e]) + bf_lo(rold[a][b][e]), bf_hi(o[e]) + bf_hi(rold[a][b][e]));
            const float h0 = bf_lo(o[e]), h1 = bf_hi(o[e]);
            ss += (m < M && n < N) ? h0 * h0 + h1 * h1 : 0.f;
          }
        }
        if (m < M && n < N) st8(out + (int64_t)m * ldo + n, o);
      }
      if (ep.res_add && ep.ss_out) {  // this wave's 32 columns of row m: the four lane groups' sums
        ss = sum_over_groups(ss);
        const int grp = (n0 + 32 * (wv & 1)) >> 5;
        if (g == 0 && m < M && n0 + 32 * (wv & 1) < N) ep.ss_out[(int64_t)(mb0 + m) * (N >> 5) + grp] = ss;
      }
    }
    return;
  }

  // k splits: the partial [S][Mall][N] goes out with sc1 stores; the tile's last workgroup to arrive sums the
  // S partials in the order s = 0 .. S-1, whichever it is (the result does not depend on the arrival order),
  // and the counter goes back to zero for the next launch
  const rsrc_t pr = make_rsrc(part, (uint32_t)((int64_t)S * Mall * N * 4));
#pragma unroll
  for (int b = 0; b < MH; ++b) {
    const int m = 16 * (im0 + b) + r16;
    if (m >= M) continue;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int n = n0 + 16 * (jn0 + a) + 4 * g;
      if (n < N)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[a][b]), pr,
                                               (uint32_t)((((int64_t)sp * Mall + mb0 + m) * N + n) * 4), 0, kSC1);
    }
  }
  __shared__ int last;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partial has reached the coherent level
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();                     // ... and every wave's
  if (threadIdx.x == 0) {
    int32_t *c = cnt + (int)blockIdx.z * (int)gridDim.x + nt;
    const int old = atomicAdd(c, 1);
    last = old == S - 1;
    if (old == S - 1) *c = 0;  // every arrival of this launch is in
  }
  __syncthreads();
  if (!last) return;
  const int ncol = min(kGmNB, N - n0) >> 3;  // 8-column groups of the tile (N is a multiple of 8)
  // (every lane runs the loop to its end: the sums of squares below reduce across lanes)
  for (int t0 = 0; t0 < M * 8; t0 += 64 * NW) {
    const int t = t0 + (int)threadIdx.x;
    const int m = min(t >> 3, M - 1), q = t & 7;
    const bool live = t < M * 8 && q < ncol;
    const int n = n0 + 8 * min(q, ncol - 1);
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const u32x4 rv = (ep.res_add && live) ? *reinterpret_cast<const u32x4 *>(out + (int64_t)m * ldo + n)
                                          : u32x4{0u, 0u, 0u, 0u};
    const uint32_t o0 = (uint32_t)((((int64_t)mb0 + m) * N + n) * 4), os = (uint32_t)((int64_t)Mall * N * 4);
    // four splits' loads in flight at a time (past S: offsets past the range, zeros, not added)
    for (int j = 0; j < S; j += 4) {
      u32x4 lo[4], hi[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t o = j + u < S ? o0 + (uint32_t)(j + u) * os : 0xFFFFFFE0u;
        lo[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, o, 0, kSC1));
        hi[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, o + 16u, 0, kSC1));
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (j + u >= S) break;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[i] += __uint_as_float(lo[u][i]);
          v[4 + i] += __uint_as_float(hi[u][i]);
        }
      }
    }
    const float iv = has_ss ? inv_s[m] : 1.f;
    u32x4 o{pack_bf16x2(v[0] * iv, v[1] * iv), pack_bf16x2(v[2] * iv, v[3] * iv), pack_bf16x2(v[4] * iv, v[5] * iv),
            pack_bf16x2(v[6] * iv, v[7] * iv)};
    if (ep.res_add) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = pack_bf16x2(bf_lo(o[e]) + bf_lo(rv[e]), bf_hi(o[e]) + bf_hi(rv[e]));
        const float h0 = bf_lo(o[e]), h1 = bf_hi(o[e]);
        ss += h0 * h0 + h1 * h1;
      }
      if (ep.ss_out) {  // a 32-column group = four consecutive lanes (q = 4j .. 4j + 3 of row m)
        ss = live ? ss : 0.f;
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        if (live && (q & 3) == 0) ep.ss_out[(int64_t)(mb0 + m) * (N >> 5) + ((n0 >> 5) + (q >> 2))] = ss;
      }
    }
    if (live) st16(out + (int64_t)m * ldo + n, o);
  }
}

bool al16g(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// 128-wide k chunks where the token tile is small (MT <= 4: twice the bytes per wait and meeting, at the same
// LDS bytes in flight) and K allows; else 64
int gm_kc(int MT, int K) { return (MT <= 4 && K % 128 == 0) ? 128 : 64; }
using GmKern = void (*)(const uint16_t *, int64_t, const uint16_t *, int64_t, uint16_t *, int64_t, float *, int32_t *,
                        int, int, int, int, int, int, GmEpi);
GmKern gm_kernel(int MT, int KC) {
  if (KC == 128) return MT == 2 ? k_gemm_small<2, 4, 128> : k_gemm_small<4, 8, 128>;
  return MT == 2 ? k_gemm_small<2, 4, 64> : MT == 4 ? k_gemm_small<4, 8, 64> : MT == 6 ? k_gemm_small<6, 4, 64>
       : MT == 8 ? k_gemm_small<8, 8, 64> : MT == 10 ? k_gemm_small<10, 4, 64> : k_gemm_small<12, 8, 64>;
}

}  // namespace
}  // namespace a8

extern "C" int a8_gemm_small(const void *x, int64_t ldx, const void *w, int64_t ldw, void *out, int64_t ldo,
                             void *ws, int64_t ws_bytes, int M, int N, int K, int splits, int mblocks, void *stream) {
  using namespace a8;
  if (M < 0 || N < 0 || K < 0 || splits < 1 || mblocks < 1)
    return set_error(A8_EINVAL, "gemm_small: bad sizes M=%d N=%d K=%d splits=%d mblocks=%d", M, N, K, splits, mblocks);
  if (M == 0 || N == 0) return 0;
  if (M > kGmMaxM || K == 0 || K % kGmKC || N % 8)
    return set_error(A8_EUNSUP, "gemm_small: M=%d N=%d K=%d outside M <= %d, K a multiple of %d, N of 8", M, N, K,
                     kGmMaxM, kGmKC);
  if (!x || !w || !out) return set_error(A8_EINVAL, "gemm_small: null pointer");
  if (!al16g(x) || !al16g(w) || !al16g(out) || (ldx | ldw | ldo) & 7 || ldx < K || ldw < K || ldo < N)
    return set_error(A8_EALIGN, "gemm_small: pointers must be 16-byte aligned, leading dims multiples of 8 and "
                     ">= the row length");
  if ((int64_t)(M - 1) * ldx * 2 + (int64_t)K * 2 >= ((int64_t)1 << 32) ||
      (int64_t)(N - 1) * ldw * 2 + (int64_t)K * 2 >= ((int64_t)1 << 32))
    return set_error(A8_EUNSUP, "gemm_small: operands span more than 4 GiB");
  const int MT = std::min(12, ((((M + mblocks - 1) / mblocks) + 31) / 32) * 2);
  const int KC = gm_kc(MT, K);
  const int nch = K / KC;
  const int S = std::min(splits, nch);
  const int cps = (nch + S - 1) / S;
  const int S_used = (nch + cps - 1) / cps;  // every split has at least one chunk
  if (S_used > 1 && (!ws || ws_bytes < kGmCntBytes + (int64_t)S_used * M * N * 4 || !al16g(ws)))
    return set_error(A8_EWSPACE, "gemm_small: %d splits need a 16-byte aligned workspace of %lld bytes", S_used,
                     (long long)(kGmCntBytes + (int64_t)S_used * M * N * 4));
  if (S_used > 1 && (int64_t)S_used * M * N * 4 >= ((int64_t)1 << 32))
    return set_error(A8_EUNSUP, "gemm_small: %d splits of %d x %d partials span more than 4 GiB", S_used, M, N);
  // rows per block: an even number of 16-row subtiles covering M / mblocks (MT above); empty blocks are dropped
  const int nmb = (M + MT * 16 - 1) / (MT * 16);
  const int ntile = (N + kGmNB - 1) / kGmNB;
  if (S_used > 1 && (int64_t)ntile * nmb > kGmCntBytes / 4)
    return set_error(A8_EUNSUP, "gemm_small: %d x %d tiles exceed the %d counters for k splits", ntile, nmb,
                     kGmCntBytes / 4);
  int32_t *cnt = S_used > 1 ? (int32_t *)ws : nullptr;
  float *part = S_used > 1 ? (float *)((char *)ws + kGmCntBytes) : nullptr;
  const dim3 grid((unsigned)ntile, (unsigned)S_used, (unsigned)nmb);
  const hipStream_t st = (hipStream_t)stream;
  // 8 waves (two per SIMD, one covering the other's LDS round trips) where the token subtiles split four ways
  const bool w8 = MT % 4 == 0;
  auto kern = gm_kernel(MT, KC);
  hipLaunchKernelGGL(kern, grid, dim3(w8 ? 512 : 256), 0, st, (const uint16_t *)x, ldx, (const uint16_t *)w, ldw,
                     (uint16_t *)out, ldo, part, cnt, M, N, K, cps, S_used, 0, GmEpi{});
  return (int)hipGetLastError();
}

extern "C" int a8_gemm_silu_small(const void *x, int64_t ldx, const void *w13, int64_t ldw, void *out, int64_t ldo,
                                  int M, int I, int K, int mblocks, void *stream) {
  using namespace a8;
  if (M < 0 || I < 0 || K < 0 || mblocks < 1)
    return set_error(A8_EINVAL, "gemm_silu_small: bad sizes M=%d I=%d K=%d mblocks=%d", M, I, K, mblocks);
  if (M == 0 || I == 0) return 0;
  if (M > kGmMaxM || K == 0 || K % kGmKC || I % 8)
    return set_error(A8_EUNSUP, "gemm_silu_small: M=%d I=%d K=%d outside M <= %d, K a multiple of %d, I of 8", M, I,
                     K, kGmMaxM, kGmKC);
  if (!x || !w13 || !out) return set_error(A8_EINVAL, "gemm_silu_small: null pointer");
  if (!al16g(x) || !al16g(w13) || !al16g(out) || (ldx | ldw | ldo) & 7 || ldx < K || ldw < K || ldo < I)
    return set_error(A8_EALIGN, "gemm_silu_small: pointers must be 16-byte aligned, leading dims multiples of 8 "
                     "and >= the row length");
  if ((int64_t)(M - 1) * ldx * 2 + (int64_t)K * 2 >= ((int64_t)1 << 32) ||
      (int64_t)(2 * I - 1) * ldw * 2 + (int64_t)K * 2 >= ((int64_t)1 << 32))
    return set_error(A8_EUNSUP, "gemm_silu_small: operands span more than 4 GiB");
  const int MT = std::min(12, ((((M + mblocks - 1) / mblocks) + 31) / 32) * 2);
  const int KC = gm_kc(MT, K);
  const int nch = K / KC;
  const int nmb = (M + MT * 16 - 1) / (MT * 16);
  const dim3 grid((unsigned)((I + 31) / 32), 1u, (unsigned)nmb);
  const bool w8 = MT % 4 == 0;
  auto kern = gm_kernel(MT, KC);
  hipLaunchKernelGGL(kern, grid, dim3(w8 ? 512 : 256), 0, (hipStream_t)stream, (const uint16_t *)x, ldx,
                     (const uint16_t *)w13, ldw, (uint16_t *)out, ldo, nullptr, nullptr, M, 2 * I, K, nch, 1, I,
                     GmEpi{});
  return (int)hipGetLastError();
}

static int gemm_small_norm_impl(const void *x, int64_t ldx, const void *w, int64_t ldw, void *out, int64_t ldo,
                                void *ws, int64_t ws_bytes, int M, int N, int K, int splits, int mblocks, int gated,
                                int res_add, float *ss_out, const float *ss_in, int ss_n, float eps, const void *pf,
                                int64_t pf_bytes, void *pf_sink, int pf_slices, void *stream) {
  using namespace a8;
  if (M < 0 || N < 0 || K < 0 || splits < 1 || mblocks < 1 || ss_n < 0)
    return set_error(A8_EINVAL, "gemm_small_norm: bad sizes M=%d N=%d K=%d splits=%d mblocks=%d", M, N, K, splits,
                     mblocks);
  if (M == 0 || N == 0) return 0;
  const int I = gated ? N / 2 : 0;  // gated: w = [gate; up] (N = 2 I rows), out [M, I]
  if (M > kGmMaxM || K == 0 || K % kGmKC || N % 8 || (gated && (N % 16 || splits != 1 || res_add)))
    return set_error(A8_EUNSUP, "gemm_small_norm: M=%d N=%d K=%d (gated %d, splits %d, res_add %d) outside M <= %d, "
                     "K a multiple of %d, N of 8 (16 gated; gated: one split, no residual)", M, N, K, gated, splits,
                     res_add, kGmMaxM, kGmKC);
  if (ss_out && (!res_add || N % 32))
    return set_error(A8_EUNSUP, "gemm_small_norm: sums of squares need res_add and N a multiple of 32 (N=%d)", N);
  if (ss_in && (ss_n < 1 || ss_n > kGmSsMax || ss_n % 4))
    return set_error(A8_EUNSUP, "gemm_small_norm: %d partial sums per row (1..%d, a multiple of 4)", ss_n, kGmSsMax);
  if (res_add && ss_in)
    return set_error(A8_EUNSUP, "gemm_small_norm: a product both adds the residual and consumes a norm");
  const int ldo_need = gated ? I : N;
  if (!x || !w || !out) return set_error(A8_EINVAL, "gemm_small_norm: null pointer");
  if (!al16g(x) || !al16g(w) || !al16g(out) || (ss_in && !al16g(ss_in)) || (ldx | ldw | ldo) & 7 || ldx < K ||
      ldw < K || ldo < ldo_need)
    return set_error(A8_EALIGN, "gemm_small_norm: pointers must be 16-byte aligned, leading dims multiples of 8 and "
                     ">= the row length");
  if ((int64_t)(M - 1) * ldx * 2 + (int64_t)K * 2 >= ((int64_t)1 << 32) ||
      (int64_t)(N - 1) * ldw * 2 + (int64_t)K * 2 >= ((int64_t)1 << 32))
    return set_error(A8_EUNSUP, "gemm_small_norm: operands span more than 4 GiB");
  const int MT = std::min(12, ((((M + mblocks - 1) / mblocks) + 31) / 32) * 2);
  const int KC = gm_kc(MT, K);
  const int nch = K / KC;
  const int S = gated ? 1 : std::min(splits, nch);
  const int cps = (nch + S - 1) / S;
  const int S_used = (nch + cps - 1) / cps;
  if (S_used > 1 && (!ws || ws_bytes < kGmCntBytes + (int64_t)S_used * M * N * 4 || !al16g(ws)))
    return set_error(A8_EWSPACE, "gemm_small_norm: %d splits need a 16-byte aligned workspace of %lld bytes", S_used,
                     (long long)(kGmCntBytes + (int64_t)S_used * M * N * 4));
  if (S_used > 1 && (int64_t)S_used * M * N * 4 >= ((int64_t)1 << 32))
    return set_error(A8_EUNSUP, "gemm_small_norm: %d splits of %d x %d partials span more than 4 GiB", S_used, M, N);
  const int nmb = (M + MT * 16 - 1) / (MT * 16);
  const int ntile = gated ? (I + 31) / 32 : (N + kGmNB - 1) / kGmNB;
  if (S_used > 1 && (int64_t)ntile * nmb > kGmCntBytes / 4)
    return set_error(A8_EUNSUP, "gemm_small_norm: %d x %d tiles exceed the %d counters for k splits", ntile, nmb,
                     kGmCntBytes / 4);
  int32_t *cnt = S_used > 1 ? (int32_t *)ws : nullptr;
  float *part = S_used > 1 ? (float *)((char *)ws + kGmCntBytes) : nullptr;
  const bool do_pf = pf && pf_bytes >= 16 && pf_slices > 0;
  if (do_pf && (!pf_sink || !al16g(pf) || !al16g(pf_sink) || pf_slices > 64))
    return set_error(A8_EINVAL, "gemm_small_norm: prefetch needs 16-byte aligned pointers and 1..64 slices");
  // pf_slices counts slices of ntile prefetch workgroups: with k splits each grid slice holds S_used times that
  const int pf_z = do_pf ? (pf_slices + S_used - 1) / S_used : 0;
  const dim3 grid((unsigned)ntile, (unsigned)S_used, (unsigned)(nmb + pf_z));
  const bool w8 = MT % 4 == 0;
  auto kern = gm_kernel(MT, KC);
  const GmEpi ep{res_add ? 1 : 0, ss_out, ss_in, ss_n, eps, do_pf ? (const u32x4 *)pf : nullptr,
                 do_pf ? pf_bytes / 16 : 0, (uint32_t *)pf_sink, nmb};
  hipLaunchKernelGGL(kern, grid, dim3(w8 ? 512 : 256), 0, (hipStream_t)stream, (const uint16_t *)x, ldx,
                     (const uint16_t *)w, ldw, (uint16_t *)out, ldo, part, cnt, M, N, K, cps, S_used, I, ep);
  return (int)hipGetLastError();
}

extern "C" int a8_gemm_small_norm(const void *x, int64_t ldx, const void *w, int64_t ldw, void *out, int64_t ldo,
                                  void *ws, int64_t ws_bytes, int M, int N, int K, int splits, int mblocks, int gated,
                                  int res_add, float *ss_out, const float *ss_in, int ss_n, float eps, void *stream) {
  return gemm_small_norm_impl(x, ldx, w, ldw, out, ldo, ws, ws_bytes, M, N, K, splits, mblocks, gated, res_add, ss_out,
                              ss_in, ss_n, eps, nullptr, 0, nullptr, 0, stream);
}

extern "C" int a8_gemm_small_norm_pf(const void *x, int64_t ldx, const void *w, int64_t ldw, void *out, int64_t ldo,
                                     void *ws, int64_t ws_bytes, int M, int N, int K, int splits, int mblocks,
                                     int gated, int res_add, float *ss_out, const float *ss_in, int ss_n, float eps,
                                     const void *pf, int64_t pf_bytes, void *pf_sink, int pf_slices, void *stream) {
  return gemm_small_norm_impl(x, ldx, w, ldw, out, ldo, ws, ws_bytes, M, N, K, splits, mblocks, gated, res_add, ss_out,
                              ss_in, ss_n, eps, pf, pf_bytes, pf_sink, pf_slices, stream);
}
