// Packed variable-length causal prefill attention over cache rows (a8_prefill_attn).
//
// Semantics follow serve/fast_kernels.py:296-358 (_prefill_attn_kernel / prefill_attention): a
// block of <= 64 packed query rows [q0, q0+n) of one request sits at positions [p0, p0+n) of cache
// row `slot`; each row attends keys [0, p0+n) of that row with key <= its position (the cached
// voice prefix [0, p0) plus the causal part of the new tokens), online softmax in fp32, bf16
// softmax weights in P.V, out = bf16(acc / l).
//
// MI355X design (compute-heavy: ~325 FLOP per compulsory byte, so both products run on MFMA):
//   * One workgroup = one query block x one kv head (x a share of its q heads when the group has more
//     than 8); its waves are the q heads (7 for the engine's GQA 7), two per SIMD, so one wave's softmax
//     VALU work overlaps the other's MFMAs. A wave reads each tile's K / V operands from LDS once and
//     runs its four 16-row query groups through them one after another (register pressure stays
//     within the 256 of two waves per SIMD).
//   * K and V tiles (64 keys x 128 B each) go from HBM / L2 straight into LDS by DMA
//     (buffer_load ... lds), double-buffered: the next tile's 16 DMA instructions (spread over the
//     waves) are in flight while the current tile is computed; one barrier per tile (each wave's own DMA
//     complete, then s_barrier) hands a tile to all waves.
//   * K is row-major with the 16-byte chunks of row r permuted by chunk ^ ((r & 3) | ((r >> 3) & 1) << 2),
//     so the permuted S^T rows (below) read 8 distinct banks per 8 lanes; V uses the decode tile's
//     layout and is read transposed by ds_read_b64_tr_b16 (decode_tile.h).
//   * Per unit: S^T = K . Q^T (v_mfma_f32_16x16x32_bf16, 64 keys x 16 query rows per tile), online
//     softmax per query column in raw score units (exp2 with the scale folded into one FMA; tiles
//     wholly below the causal diagonal skip the mask; the accumulator rescale is skipped when no max
//     moved), O^T += V^T . P^T with the S^T C-layout reused as the P^T B operand (key rows permuted
//     within 32-key chunks, as in the decode kernel).
#include <type_traits>

#include "decode_tile.h"
#include "rope.h"

namespace a8 {

constexpr int kPfMaxHW = 4;   // q heads (waves) per workgroup: two workgroups fit a compute unit's LDS
constexpr float kPfLazy = 8.f;  // exp2 units a column's running max may lag behind its scores
constexpr float kPfLow = -64.f;  // on a block's first tile: a column max below this sets the offset (underflow)

// K chunk permutation of tile row r (see above).
__device__ __forceinline__ int pf_kswz(int r) { return (r & 3) | (((r >> 3) & 1) << 2); }

// Requests DMA instruction i (0..15) of tile rows [t0, t0 + 64): i < 8 K rows 8i..8i+7, else V rows
// 8(i-8).. . k0 / k1, v0 / v1: this lane's source offsets inside a tile for even / odd instructions
// (plain values: i depends on the wave, and an array indexed by it would live in scratch memory).
__device__ __forceinline__ void pf_dma(int i, uint32_t t0, rsrc_t kr, rsrc_t vr, uint16_t *kt, uint16_t *vt,
                                       uint32_t k0, uint32_t k1, uint32_t v0, uint32_t v1) {
  const int j = i & 7;
  const uint32_t off = t0 * kRow + (uint32_t)j * 1024u;
  const bool odd = j & 1;
  if (i < 8)
    bld16_lds<0>(kr, reinterpret_cast<char *>(kt) + j * 1024, off + (odd ? k1 : k0), 0u);
  else
    bld16_lds<0>(vr, reinterpret_cast<char *>(vt) + j * 1024, off + (odd ? v1 : v0), 0u);
}

// The query operands formed from the qkv rows (a8_prefill_attn_qkv): bias and RoPE tables; unused otherwise.
struct PfQkv {
  const uint16_t *bias, *cos_tab, *sin_tab;
  int64_t s_cs;
  int n_tab;
};

// UPW = 16-row query groups per wave (the block's 64 rows).
constexpr int UPW = 4;
// NW = waves (q heads) per workgroup, 1..kPfMaxHW. QKV: q / s_qr / s_qh address the q columns of the qkv rows
// (s_qh = the head dimension) and the query operands are formed from them with qk's bias and tables.
template <int NW, bool QKV>
__global__ __launch_bounds__(64 * kPfMaxHW, 2) void k_prefill(
    const uint16_t *__restrict__ q, int64_t s_qr, int64_t s_qh, int R,
    const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
    int cache_rows, int cache_len, uint16_t *__restrict__ out, int64_t s_or, int64_t s_oh,
    const int32_t *__restrict__ bq0, const int32_t *__restrict__ bn, const int32_t *__restrict__ bslot,
    const int32_t *__restrict__ bpos0, int group, int hsplit, int hpw, float sl2, int nh, int nblk_, PfQkv qk) {
  warm_kernargs<200>();  // the explicit arguments above span 0x00-0xc7
  // a ring of three K and three V tile buffers (tiles are requested two ahead), separate arrays so the
  // compiler tells their DMA apart
  __shared__ __attribute__((aligned(16))) uint16_t kA[kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t kB[kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t kC[kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t vA[kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t vB[kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t vC[kVTile];
  // Q^T operands of every wave's query groups, parked in LDS (8 KB per wave) to keep registers for the
  // accumulators: [wave][group][dim half][lane] x 16 bytes
  __shared__ __attribute__((aligned(16))) uint16_t qs[kPfMaxHW * 4 * 2 * 64 * 8];
  // Workgroups in unit order, unit u = (block, kv head) = blk * nkv + kh, so a plan that lists its heaviest
  // blocks first is dispatched heaviest-first; the hsplit head shares of a unit are 8 workgroups apart, so
  // they land on one XCD (workgroup i runs on XCD i % 8) and the second reads the unit's tiles from that
  // XCD's L2 (C4: 42.0 -> 41.7 us against adjacent shares on neighbouring XCDs). The grid is padded to whole
  // runs of 8 units; workgroups past the last unit exit at once.
  const int nkv_ = nh / hsplit;
  const int chunk = blockIdx.x / (8 * hsplit), rem = blockIdx.x - chunk * (8 * hsplit);
  const int hs = rem >> 3, u = chunk * 8 + (rem & 7);
  const int blk = u / nkv_, kh = u - blk * nkv_;
  if (blk >= nblk_) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int nw = NW;
  const int r16 = lane & 15, g = lane >> 4;

  // Block metadata is uniform over the workgroup, so early exits happen before any barrier.
  const int n = bn[blk];
  if (n <= 0) return;  // graph-mode padding block
  const int q0 = bq0[blk], p0 = bpos0[blk];
  const int64_t sl = bslot[blk];
  if (sl < 0 || sl >= cache_rows || p0 < 0 || q0 < 0 || q0 >= R) return;
  const int nv = min(min(n, 64), R - q0);  // valid query rows
  const int hi = min(p0 + n, cache_len);   // keys [0, hi)
  if (hi <= 0) return;
  const int ntile = (hi + 63) / 64;

  // K / V of this (cache row, kv head) as buffers ending at key hi: rows past it read as zeros.
  const int64_t cb = sl * s_kb + (int64_t)kh * s_kh;
  const rsrc_t kr = make_rsrc(kc + cb, (uint32_t)hi * kRow);
  const rsrc_t vr = make_rsrc(vc + cb, (uint32_t)hi * kRow);
  TileLane tl;
  tl.init(lane);
  const int row8 = lane >> 3, ch8 = lane & 7;
  const uint32_t kd0 = (uint32_t)row8 * kRow + 16u * (uint32_t)(ch8 ^ (row8 & 3));
  const uint32_t kd1 = (uint32_t)row8 * kRow + 16u * (uint32_t)(ch8 ^ ((row8 & 3) | 4));
  const uint32_t vd0 = tl.vd[0], vd1 = tl.vd[1];
  uint32_t vt[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) vt[dt] = tl.vt[dt];
  // K A-operand reads: row 32c + 8(r16/4) + 4t + r16%4, chunk g (+4 for dims 32..63)
  const int krow = 8 * (r16 >> 2) + (r16 & 3), kz = pf_kswz(krow);
  const uint32_t ko0 = (uint32_t)krow * kRow + 16u * (uint32_t)(g ^ kz);
  const uint32_t ko1 = (uint32_t)krow * kRow + 16u * (uint32_t)((4 + g) ^ kz);

  // This wave's units k = query group qt (rows 16k..16k+15 of the block) of q head hs*hpw + w.
  const int gi = hs * hpw + w;
  const bool active = gi < group;
  bool live[UPW];
  int head[UPW], qt_of[UPW];
  // Q^T operands: column r16 <-> query row 16qt + r16, slot (g, j) <-> dim 8g+j / 32+8g+j
  uint16_t *qw = qs + w * (4 * 2 * 64 * 8) + lane * 8;
  f32x4 o[UPW][4];   // O^T rows d = 16dt + 4g + i, column = query row 16qt + r16
  // per query group: the exp2 offset mcs (in exp2 units, 0 to start with; see the raise below)
  float mcs[UPW];
  f32x4 cneg[UPW];  // {-mcs} x 4: the score products' C operand, kept in registers
  f32x4 lacc[UPW];  // column sums of the weights (all four rows alike)
  // bf16 1.0 pairs, made once by an opaque move so that the compiler keeps them in registers (it would
  // otherwise rebuild the constant before every group's row-sum products)
  u32x4 ones;
  asm volatile("v_mov_b32 %0, 0x3f803f80" : "=v"(ones[0]));
  ones[1] = ones[0];
  ones[2] = ones[0];
  ones[3] = ones[0];
  // The Q^T operands go from HBM straight into LDS by DMA (requested before the first K / V tiles, so the
  // first wait covers both): lane l of request (k, half) reads dims 8g.. (+32) of query row 16k + r16, and
  // rows past nv read as zeros (the descriptor ends at row nv - 1; the host keeps s_qr >= hd).
  // QKV: the same chunks of the qkv rows, the bias chunks and the tables' chunks at each row's position go to
  // registers instead (before the first K / V requests; formed into the operands after them).
  u32x4 qx[UPW][2], qcs[UPW][4], qb[2];
  if (active) {
    const rsrc_t qrs = make_rsrc(q + (int64_t)q0 * s_qr + (int64_t)(kh * group + gi) * s_qh,
                                 (uint32_t)((int64_t)(nv - 1) * s_qr * 2 + 128));
    if constexpr (QKV) {
      const int hq = kh * group + gi;
      // every operand through a buffer of its own extent (the host keeps n_tab x s_cs x 2 below 2^32):
      // a position past the tables, or no bias, reads zeros
      const rsrc_t br = make_rsrc(qk.bias, qk.bias ? (uint32_t)((hq + 1) * 128) : 0u);
      const uint32_t tab = (uint32_t)((int64_t)qk.n_tab * qk.s_cs * 2);
      const rsrc_t cr = make_rsrc(qk.cos_tab, tab), sr = make_rsrc(qk.sin_tab, tab);
      qb[0] = bld16(br, (uint32_t)(hq * 128 + 16 * g));
      qb[1] = bld16(br, (uint32_t)(hq * 128 + 64 + 16 * g));
#pragma unroll
      for (int k = 0; k < UPW; ++k) {
        qx[k][0] = bld16(qrs, (uint32_t)(((int64_t)(16 * k + r16) * s_qr + 8 * g) * 2));
        qx[k][1] = bld16(qrs, (uint32_t)(((int64_t)(16 * k + r16) * s_qr + 8 * g + 32) * 2));
        const int p = p0 + 16 * k + r16;  // >= 0 (p0 is)
        const uint32_t co = p < qk.n_tab ? (uint32_t)((int64_t)p * qk.s_cs * 2) : tab;
        qcs[k][0] = bld16(cr, co + 16u * g);
        qcs[k][1] = bld16(cr, co + 64u + 16u * g);
        qcs[k][2] = bld16(sr, co + 16u * g);
        qcs[k][3] = bld16(sr, co + 64u + 16u * g);
      }
    } else {
#pragma unroll
      for (int k = 0; k < UPW; ++k)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          bld16_lds<0>(qrs, reinterpret_cast<char *>(qs) + (w * 8 + 2 * k + h) * 1024,
                       (uint32_t)(((int64_t)(16 * k + r16) * s_qr + 8 * g + 32 * h) * 2), 0u);
    }
  }
#pragma unroll
  for (int k = 0; k < UPW; ++k) {
    live[k] = active;
    head[k] = kh * group + gi;
    qt_of[k] = k;
    mcs[k] = 0.f;
    cneg[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    lacc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[k][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // this wave's share of a tile's 16 DMA instructions
  auto issue = [&](int t, uint16_t *kt, uint16_t *vt) __attribute__((always_inline)) {
    for (int i = w; i < 16; i += nw) pf_dma(i, (uint32_t)(64 * t), kr, vr, kt, vt, kd0, kd1, vd0, vd1);
  };
  // tile t requested by every wave: this wave's share of it complete (with the next tile's share still in
  // flight when `ahead`: loads complete in order and every wave issues at least 16 / nw instructions a
  // tile, so at most that many may stay outstanding), then meet -- which also retires every wave's LDS
  // reads of the buffer the next request will refill.
  auto ready = [&](bool ahead) __attribute__((always_inline)) {
    if (ahead) {
      if (nw == 1) __builtin_amdgcn_s_waitcnt(0x4F70);  // s_waitcnt vmcnt(16 / nw)
      if (nw == 2) __builtin_amdgcn_s_waitcnt(0x0F78);
      if (nw == 3) __builtin_amdgcn_s_waitcnt(0x0F75);
      if (nw == 4) __builtin_amdgcn_s_waitcnt(0x0F74);
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    lds_barrier();
  };
  // Scores in exp2 units: the Q^T operands are pre-scaled by sl2 = scale * log2(e) once per block (rounded to
  // bf16) and the score products start from -mcs (the MFMA's C operand), so S = q.k * sl2 - mcs comes out of the
  // matrix cores and a weight is one v_exp_f32 (no FMA per score). Lazy running maximum: a column's offset is
  // raised only when a tile's score exceeds it by more than kPfLazy, so most tiles skip the accumulator
  // rescale; until then its weights stay below 2^kPfLazy (well inside bf16's range; the sums are fp32). Same
  // softmax; the roundings happen at other points (q * sl2 once in bf16 instead of the product in fp32). C4, one
  // box: 43.7 -> 43.2 us per layer against the FMA per score.
  auto c0 = [&](int k) __attribute__((always_inline)) { return cneg[k]; };
  // S^T of query group k against the tile's K rows (8 MFMAs)
  auto scores = [&](int k, const u32x4 (&ka)[2][2][2], f32x4 (&s)[2][2]) __attribute__((always_inline)) {
    const u32x4 qb0 = ld16(qw + (2 * k) * 64 * 8), qb1 = ld16(qw + (2 * k + 1) * 64 * 8);
    const f32x4 ci = c0(k);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) s[c][tt] = mfma16x16x32(ka[c][tt][1], qb1, mfma16x16x32(ka[c][tt][0], qb0, ci));
  };
  // O^T += V^T . P^T for query group k, and the weights' column sums by the same products with a ones
  // operand (10 MFMAs, no VALU adds)
  auto weigh = [&](int k, const u32x4 (&va)[4][2], const u32x4 (&pB)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int c = 0; c < 2; ++c) o[k][dt] = mfma16x16x32(va[dt][c], pB[c], o[k][dt]);
    lacc[k] = mfma16x16x32(ones, pB[1], mfma16x16x32(ones, pB[0], lacc[k]));
  };
  // One tile. The four query groups are software-pipelined: while group k's softmax runs on the VALU,
  // the matrix cores compute group k+1's scores and group k-1's products (the scheduler is asked to
  // interleave them), so one wave keeps both units busy. MASKED: a tile that crosses the causal diagonal
  // or the range end; the two kinds run in separate loops (all full tiles first), so no scores move
  // between registers for a shared continuation.
  // ISSUE: tile tn's requests (into kn / vn) go out from inside the computation, this wave's share a
  // quarter at a time at the start of each query group, so the load queue of the compute unit drains
  // between them instead of holding every wave at once behind a burst right after the barrier. A tile past
  // the range (tn >= ntile) reads as zeros into a buffer no later tile uses: requested anyway, so no
  // branch splits the scheduled code.
  auto compute = [&](auto masked_tag, int t, const uint16_t *kt, const uint16_t *vtile, auto issue_tag, int tn,
                     uint16_t *kn, uint16_t *vn) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool ISSUE = decltype(issue_tag)::value;
    if (!active) {
      if (ISSUE) issue(tn, kn, vn);
      return;
    }
    const int kt0 = 64 * t;
    // operands of the tile, read once: K rows (A of S^T; tile (c, tt) row 4g+i <-> key
    // kt0 + 32c + 8g + 4tt + i) and V^T (A of O^T)
    u32x4 ka[2][2][2], va[4][2];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const char *kp = reinterpret_cast<const char *>(kt) + (32 * c + 4 * tt) * kRow;
        ka[c][tt][0] = ld16(kp + ko0);
        ka[c][tt][1] = ld16(kp + ko1);
      }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const char *vp = reinterpret_cast<const char *>(vtile) + vt[dt] + 32 * c * kRow;
        const u32x2 lo = lds_tr16(vp), hi2 = lds_tr16(vp + 4 * kRow);
        va[dt][c] = u32x4{lo[0], lo[1], hi2[0], hi2[1]};
      }
    f32x4 s[2][2];
    u32x4 pP[2];  // the previous group's weights
    scores(0, ka, s);
#pragma unroll
    for (int k = 0; k < UPW; ++k) {
      if (ISSUE)  // this wave's instructions i = w + nw * j with j = k mod 4 (no branch unless nw is 3)
#pragma unroll
        for (int j = k; j * nw < 16; j += 4)
          if (nw != 3 || w + nw * j < 16) pf_dma(w + nw * j, (uint32_t)(64 * tn), kr, vr, kn, vn, kd0, kd1, vd0, vd1);
      // group k+1's Q^T operands, early enough for its score products below
      u32x4 qn0, qn1;
      if (k + 1 < UPW) {
        qn0 = ld16(qw + (2 * k + 2) * 64 * 8);
        qn1 = ld16(qw + (2 * k + 3) * 64 * 8);
      }
      if (MASKED) {
        // keys <= query position (and < hi): key kt0 + 8g + off of this lane, off = 32c + 4tt + i, against
        // one threshold per lane (16 compares with constants)
        const int d = min(p0 + 16 * qt_of[k] + r16, hi - 1) - kt0 - 8 * g;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (32 * c + 4 * tt + i > d) s[c][tt][i] = kNegInf;
      }
      // group k's column max on the VALU, one step beside each of group k-1's products (the
      // scheduling barriers keep the interleave: a wave issues in order, so a run of MFMAs would stall
      // it while the VALU idles)
      // (as a tree of depth three: five independent triples, then two, then one)
      const float *sf = reinterpret_cast<const float *>(&s[0][0]);
      float mA[5], mB0 = 0.f, mB1 = 0.f, mt = 0.f;
#pragma unroll
      for (int j = 0; j < 7; ++j) {
        if (k > 0) {
          const int dt = j >> 1, c = j & 1;
          o[k - 1][dt] = mfma16x16x32(va[dt][c], pP[c], o[k - 1][dt]);
        }
        if (j < 2) {
          mA[2 * j] = max3_ieee(sf[6 * j], sf[6 * j + 1], sf[6 * j + 2]);
          mA[2 * j + 1] = max3_ieee(sf[6 * j + 3], sf[6 * j + 4], sf[6 * j + 5]);
        } else if (j == 2) {
          mA[4] = max3_ieee(sf[12], sf[13], sf[14]);
        } else if (j == 3) {
          mB0 = max3_ieee(mA[0], mA[1], mA[2]);
        } else if (j == 4) {
          mB1 = max3_ieee(mA[3], mA[4], sf[15]);
        } else if (j == 5) {
          mt = max_ieee(mB0, mB1);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (k > 0) {
        o[k - 1][3] = mfma16x16x32(va[3][1], pP[1], o[k - 1][3]);
        lacc[k - 1] = mfma16x16x32(ones, pP[1], mfma16x16x32(ones, pP[0], lacc[k - 1]));
      }
      // mt is this lane group's max (16 of the column's 64 scores). The offset starts at 0 and is raised only
      // when some lane group of some column passes it by more than kPfLazy (its weights stay below 2^kPfLazy;
      // the column max is formed only then). On the block's first tile -- key 0 is visible to every row, so
      // every column has a key there -- it is also set when a lane group's max is below kPfLow, so that a
      // column's weights cannot all underflow (fp32 reaches 2^-126): a column's largest weight stays in
      // [2^kPfLow, 2^kPfLazy]. With ordinary scores no raise happens on the first tile (it used to take the
      // first tile's max as the offset in every group).
      const bool first = kt0 == 0;
      if (__ballot(mt > kPfLazy || mt < (first ? kPfLow : kNegInf))) {
        // t: the column's max relative to its offset; on the first tile it becomes the offset (nothing has
        // accumulated yet), later the offset moves up by max(t, 0); the tile's scores and the accumulators
        // follow.
        const float t = max_over_groups_ieee(mt);
        const float up = first ? t : fmaxf(t, 0.f);
        const float alpha = first ? 0.f : fast_exp2(-up);
        lacc[k] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[k][dt] *= alpha;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) s[c][tt] -= up;
        mcs[k] += up;
        cneg[k] = f32x4{-mcs[k], -mcs[k], -mcs[k], -mcs[k]};
      }
      // group k's weights on the VALU, one score product of group k+1 beside each quarter tile
      f32x4 sn[2][2];
      u32x4 pB[2];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          if (k + 1 < UPW) sn[c][tt] = mfma16x16x32(ka[c][tt][0], qn0, c0(k + 1));
          float pv[4];
          pv[0] = fast_exp2(s[c][tt][0]);
          pv[1] = fast_exp2(s[c][tt][1]);
          pB[c][2 * tt] = pack_bf16x2(pv[0], pv[1]);
          __builtin_amdgcn_sched_barrier(0);
          if (k + 1 < UPW) sn[c][tt] = mfma16x16x32(ka[c][tt][1], qn1, sn[c][tt]);
          pv[2] = fast_exp2(s[c][tt][2]);
          pv[3] = fast_exp2(s[c][tt][3]);
          pB[c][2 * tt + 1] = pack_bf16x2(pv[2], pv[3]);
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        pP[c] = pB[c];
        if (k + 1 < UPW)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) s[c][tt] = sn[c][tt];
      }
    }
    weigh(UPW - 1, va, pP);
  };

  // tiles [0, nfull) lie wholly below the causal diagonal (every query row sees every key) and inside the
  // range; the rest -- at most two, as a block holds at most 64 positions -- cross it. Tile t sits in
  // buffer t % 3; tiles t + 1 and t + 2 are in flight while t is computed.
  const int nfull = min(max((p0 + 1) / 64, 0), hi / 64);
  issue(0, kA, vA);
  if (ntile > 1) issue(1, kB, vB);
  // the Q^T operands times sl2, rounded to bf16, in place, once their DMA has landed (it went out before this
  // wave's share of tile 0: at least 16 / NW requests after it). QKV: the operands are the q bias_rope_store
  // writes (rope.h, the store kernel's arithmetic, with the same bits for every non-NaN input; zeros for rows
  // past nv and positions outside the tables), then scaled alike and written to the same LDS slots.
  if (active) {
    auto scale = [&](u32x4 v) __attribute__((always_inline)) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = pack_bf16x2(bf_lo(v[e]) * sl2, bf_hi(v[e]) * sl2);
      return v;
    };
    if constexpr (QKV) {
#pragma unroll
      for (int k = 0; k < UPW; ++k) {
        float xl[8], xh[8];
        u32x4 olo, ohi;
        float ol[8], oh[8];
        rope_x(qx[k][0], qx[k][1], qb[0], qb[1], qk.bias != nullptr, xl, xh);
        rope_rotate_f(xl, xh, qcs[k][0], qcs[k][1], qcs[k][2], qcs[k][3], ol, oh);
        // narrowed by the hardware conversion (round to nearest even: the store's bits for every non-NaN
        // value, at one instruction per pair)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          olo[e] = pack_bf16x2(ol[2 * e], ol[2 * e + 1]);
          ohi[e] = pack_bf16x2(oh[2 * e], oh[2 * e + 1]);
        }
        const int mrow = 16 * k + r16, p = p0 + mrow;
        const bool ok = mrow < nv && p < qk.n_tab;
        const u32x4 z{0u, 0u, 0u, 0u};
        st16(qw + (2 * k) * 64 * 8, ok ? scale(olo) : z);
        st16(qw + (2 * k + 1) * 64 * 8, ok ? scale(ohi) : z);
      }
    } else {
      wait_vmcnt<16 / NW>();
#pragma unroll
      for (int j = 0; j < 2 * UPW; ++j) {
        uint16_t *p = qw + j * 64 * 8;
        st16(p, scale(ld16(p)));
      }
    }
  }
  // Wave priority (s_setprio, inside this workgroup's waves; no stream priority): 1 while more than half of
  // the block's tiles remain, 0 after. Of two workgroups on a SIMD the one further from its end is issued
  // first, so a workgroup that has just started is not held back by one about to finish (measured at C4: a
  // workgroup that starts second on a compute unit ran at half the other's tile rate, and the refills of the
  // freed slots spread the kernel's tail; 41.8 -> 40.5 us per layer; priority by the block's total tiles
  // instead: 42.6).
  auto prio = [&](int rem) __attribute__((always_inline)) {
    if (2 * rem > ntile) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
  };
  int t = 0;
  if (nfull > 0) {
    for (;; t += 3) {
      prio(ntile - t);
      ready(t + 1 < ntile);
      compute(std::false_type{}, t, kA, vA, std::true_type{}, t + 2, kC, vC);
      if (t + 1 >= nfull) {
        t += 1;
        break;
      }
      prio(ntile - t - 1);
      ready(t + 2 < ntile);
      compute(std::false_type{}, t + 1, kB, vB, std::true_type{}, t + 3, kA, vA);
      if (t + 2 >= nfull) {
        t += 2;
        break;
      }
      prio(ntile - t - 2);
      ready(t + 3 < ntile);
      compute(std::false_type{}, t + 2, kC, vC, std::true_type{}, t + 4, kB, vB);
      if (t + 3 >= nfull) {
        t += 3;
        break;
      }
    }
  }
  // the diagonal tiles: every request has gone out (t + 2 >= ntile here), so one instantiation with the
  // buffer picked at run time costs no overlap
  for (; t < ntile; ++t) {
    prio(ntile - t);
    ready(false);
    const int bsel = t % 3;
    const uint16_t *kt = bsel == 0 ? kA : bsel == 1 ? kB : kC;
    const uint16_t *vtb = bsel == 0 ? vA : bsel == 1 ? vB : vC;
    compute(std::true_type{}, t, kt, vtb, std::false_type{}, 0, kA, vA);
  }
  // the last request may still write (zeros, past the range) into LDS: let it land before the end
  __builtin_amdgcn_s_waitcnt(0x0F70);

#pragma unroll
  for (int k = 0; k < UPW; ++k) {
    if (!live[k]) continue;
    const int mrow = 16 * qt_of[k] + r16;
    if (mrow >= nv) continue;
    // a live row has l >= 2^kPfLow (its largest weight is 2^kPfLow .. 2^kPfLazy): one hardware reciprocal
    // (1 ulp) instead of sixteen IEEE divisions
    const float rl = __builtin_amdgcn_rcpf(lacc[k][0]);
    uint16_t *op = out + (int64_t)(q0 + mrow) * s_or + (int64_t)head[k] * s_oh + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      st8(op + 16 * dt, u32x2{pack_bf16x2(o[k][dt][0] * rl, o[k][dt][1] * rl),
                              pack_bf16x2(o[k][dt][2] * rl, o[k][dt][3] * rl)});
  }
}

static inline bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace a8

namespace a8 {
// Body of a8_prefill_attn and a8_prefill_attn_qkv (qk non-null: q / s_qr address the qkv rows' q columns).
static int prefill_entry(const char *fn, const void *q, int64_t s_qr, int64_t s_qh, int R, const void *kc,
                         const void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks, int cache_rows, int cache_len,
                         void *out, int64_t s_or, int64_t s_oh, const int32_t *bq0, const int32_t *bn,
                         const int32_t *bslot, const int32_t *bpos0, int nblk, int bm, int nq, int group, int hd,
                         float scale, const PfQkv *qk, void *stream) {
  if (hd != 64 && (qk || hd != 128))
    return set_error(A8_EUNSUP, "%s: head_dim %d not supported (64%s)", fn, hd, qk ? "" : " or 128");
  if (bm != 64) return set_error(A8_EUNSUP, "%s: block size %d not supported (64 only)", fn, bm);
  if (nblk < 0 || R < 0 || nq <= 0 || group <= 0 || nq % group || cache_rows < 0 || cache_len < 0)
    return set_error(A8_EINVAL, "%s: bad sizes nblk=%d R=%d nq=%d group=%d", fn, nblk, R, nq, group);
  if (qk && (qk->n_tab < 0 || qk->s_cs < hd))
    return set_error(A8_EINVAL, "%s: bad tables n_tab=%d s_cs=%lld", fn, qk->n_tab, (long long)qk->s_cs);
  if (qk && (int64_t)qk->n_tab * qk->s_cs * 2 >= (int64_t)UINT32_MAX - 256)  // the tables' 32-bit byte offsets
    return set_error(A8_EUNSUP, "%s: RoPE tables of %d x %lld too large", fn, qk->n_tab, (long long)qk->s_cs);
  if (nblk == 0 || R == 0) return 0;
  if (!q || !kc || !vc || !out || !bq0 || !bn || !bslot || !bpos0 || (qk && (!qk->cos_tab || !qk->sin_tab)))
    return set_error(A8_EINVAL, "%s: null pointer", fn);
  if (!al16(q) || !al16(kc) || !al16(vc) || !al16(out) || (s_qr | s_qh | s_kb | s_kh | s_ks | s_or | s_oh) & 7 ||
      (qk && (!al16(qk->cos_tab) || !al16(qk->sin_tab) || (qk->bias && !al16(qk->bias)) || (qk->s_cs & 7))))
    return set_error(A8_EALIGN, "%s: pointers must be 16-byte aligned and strides multiples of 8", fn);
  if (s_ks != hd)
    return set_error(A8_EUNSUP, "%s: cache positions must be contiguous rows (s_ks %lld)", fn, (long long)s_ks);
  const int nkv = nq / group;
  if (hd != 64)  // head_dim 128 (prefill128.hip)
    return prefill128(q, s_qr, s_qh, R, kc, vc, s_kb, s_kh, cache_rows, cache_len, out, s_or, s_oh, bq0, bn, bslot,
                      bpos0, nblk, nq, group, scale, (hipStream_t)stream);
  const int hpw = group < kPfMaxHW ? group : kPfMaxHW;  // q heads (waves) per workgroup
  const int hsplit = (group + hpw - 1) / hpw;
  const int nh = nkv * hsplit;
  if (s_qr < hd || s_qr >= (1 << 25))  // the Q requests' 32-bit byte offsets (63 rows) and their row range
    return set_error(A8_EUNSUP, "%s: q row stride %lld outside [%d, 2^25)", fn, (long long)s_qr, hd);
  const int64_t grid = ((int64_t)nblk * nkv + 7) / 8 * 8 * hsplit;  // whole runs of 8 units (see k_prefill)
  if (grid * 64 * hpw > (int64_t)UINT32_MAX)  // the launch counts its threads in 32 bits
    return set_error(A8_EUNSUP, "%s: too many blocks x heads (%d x %d)", fn, nblk, nh);
  static_assert(kPfMaxHW == 4, "one instantiation per workgroup size");
  const PfQkv none{nullptr, nullptr, nullptr, 0, 0};
  auto kern = qk ? (hpw == 1 ? k_prefill<1, true> : hpw == 2 ? k_prefill<2, true> : hpw == 3 ? k_prefill<3, true>
                                                                                            : k_prefill<4, true>)
                 : (hpw == 1 ? k_prefill<1, false> : hpw == 2 ? k_prefill<2, false> : hpw == 3 ? k_prefill<3, false>
                                                                                             : k_prefill<4, false>);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * hpw), 0, (hipStream_t)stream,
                     (const uint16_t *)q, s_qr, s_qh, R, (const uint16_t *)kc, (const uint16_t *)vc, s_kb, s_kh, s_ks,
                     cache_rows, cache_len, (uint16_t *)out, s_or, s_oh, bq0, bn, bslot, bpos0, group, hsplit, hpw,
                     scale * kLog2e, nh, nblk, qk ? *qk : none);
  return (int)hipGetLastError();
}
}  // namespace a8

extern "C" int a8_prefill_attn(const void *q, int64_t s_qr, int64_t s_qh, int R,
                               const void *kc, const void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                               int cache_rows, int cache_len,
                               void *out, int64_t s_or, int64_t s_oh,
                               const int32_t *bq0, const int32_t *bn, const int32_t *bslot,
                               const int32_t *bpos0, int nblk, int bm,
                               int nq, int group, int hd, float scale, void *stream) {
  return a8::prefill_entry("prefill_attn", q, s_qr, s_qh, R, kc, vc, s_kb, s_kh, s_ks, cache_rows, cache_len, out,
                           s_or, s_oh, bq0, bn, bslot, bpos0, nblk, bm, nq, group, hd, scale, nullptr, stream);
}

extern "C" int a8_prefill_attn_qkv(const void *qkv, int64_t s_qkv, const void *bias,
                                   const void *cos_tab, const void *sin_tab, int64_t s_cs, int n_tab, int R,
                                   const void *kc, const void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                                   int cache_rows, int cache_len,
                                   void *out, int64_t s_or, int64_t s_oh,
                                   const int32_t *bq0, const int32_t *bn, const int32_t *bslot,
                                   const int32_t *bpos0, int nblk, int bm,
                                   int nq, int group, int hd, float scale, void *stream) {
  const a8::PfQkv qk{(const uint16_t *)bias, (const uint16_t *)cos_tab, (const uint16_t *)sin_tab, s_cs, n_tab};
  return a8::prefill_entry("prefill_attn_qkv", qkv, s_qkv, hd, R, kc, vc, s_kb, s_kh, s_ks, cache_rows, cache_len,
                           out, s_or, s_oh, bq0, bn, bslot, bpos0, nblk, bm, nq, group, hd, scale, &qk, stream);
}
