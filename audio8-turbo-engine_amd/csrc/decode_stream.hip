// Streaming split-K decode (a8_decode_attn_stream, a8_decode_choose_stream): the default launch of the
// decode attention of serve/fast_kernels.py:193-290 on MI355X.
//
// Same semantics as the split + combine pair (decode.hip): query row b attends keys [0, lens[b]) of
// cache row rowmap[b] with an fp32 online softmax and bf16 softmax weights in P.V, and the partial
// results over key ranges are merged with w = exp(m - M). What changes is the schedule, chosen for
// HBM3E (measured on MI355X: a 201 MB read issued as a few hundred independent 256-KB streams runs
// ~10 % slower than the same bytes swept in address order, and a separate combine launch costs
// 3-4 us per layer):
//   * Work unit = chunk of CH = waves * tpw * 64 keys of one (row, kv head); a unit (row, kv head)
//     has P = ceil(cache_len / CH) chunks, numbered in cache address order. A persistent grid of G
//     workgroups takes chunks g, g + G, g + 2G, ... so the GPU as a whole sweeps the cache in address
//     order through a window of about G * CH * 256 bytes.
//   * Inside a chunk the workgroup's waves take 64-key tiles round-robin (decode_tile.h); each wave
//     keeps a two-tile register pipeline that runs across chunk boundaries, so the next chunk's
//     loads are in flight while a chunk's partials are merged and written.
//   * Per chunk the waves' partials are merged in LDS (double-buffered, one barrier per chunk), each
//     wave merging a share of the outputs (one wave doing all of it costs ~5 us per layer: the next
//     chunk's barrier waits for it). A row whose keys fit in one chunk is
//     written straight to `out`; otherwise the merging wave stores the chunk's (acc, m, l) to the
//     workspace and moves on, and k_decode_stream_combine (launched right after, one thread per
//     output element) merges the row's chunks. Merging inside the streaming kernel instead would
//     need a device-scope handshake per chunk (store completion, counter atomic, partial reads): on a
//     saturated memory system each of those round trips waits microseconds in the same queues the
//     KV stream fills, which costs far more than the extra launch.
#include "decode_tile.h"
#include "rope.h"

namespace a8 {

// NT = 64-key tiles per pipeline step (decode_tile.h compute_step); tpw is a multiple of NT. With
// NT = 2, or FUSED (the next chunk's qkv / bias / table chunks are held in registers), a wave may use
// up to 512 registers (one wave per SIMD).
// FUSED: q and the new k / v come from qkv + bias + RoPE (rope.h, the store kernel's arithmetic) at each
// chunk's first step instead of from q; the unit's first chunk stores k / v (and q) like
// k_bias_rope_store, and the tile holding the new key column takes it from registers.
template <int NW, int NT, bool FUSED>
__global__ __launch_bounds__(64 * NW, (NT == 1 && !FUSED) ? 2 : 1) void k_decode_stream(
    const uint16_t *__restrict__ q, int64_t s_qb, int64_t s_qh,
    uint16_t *kc, uint16_t *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,  // written when FUSED
    int cache_rows, int cache_len, const int32_t *__restrict__ lens, const int32_t *__restrict__ rowmap,
    uint16_t *__restrict__ out, int64_t s_ob, int64_t s_oh, float *__restrict__ acc_ws,
    float *__restrict__ ml_ws, int b, int nq, int nkv, int group, int tpw, int P,
    float sl2, StoreIn si) {
  warm_kernargs<264>();  // the explicit arguments above span 0x000-0x10f
  // V tiles of the two pipeline buffers (NT per wave each). A step reads its tiles after a counted
  // vmcnt wait: the next step's 16 NT requests are issued before it.
  __shared__ __attribute__((aligned(16))) uint16_t vbA[NW * NT * kVTile];
  __shared__ __attribute__((aligned(16))) uint16_t vbB[NW * NT * kVTile];
  __shared__ __attribute__((aligned(16))) float mrg[2][NW * (32 + 16 * kOb)];  // per-wave m, l, O (x2)
  __shared__ int marr[2], mseq[2];  // per merge buffer: waves arrived, last merge completed

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x;
  const int CH = NW * tpw * 64;
  const int NC = b * nkv * P;
  const int nmine = ((int)blockIdx.x < NC) ? (NC - 1 - (int)blockIdx.x) / G + 1 : 0;
  if (nmine == 0) return;
  if (tid < 2) {
    marr[tid] = 0;
    mseq[tid] = tid - 2;
  }
  lds_barrier();

  constexpr uint32_t row_bytes = kRow;  // s_ks == 64, checked by the entry point
  const uint32_t full_row = (uint32_t)cache_len * row_bytes;
  TileLane tl;
  tl.init(lane);
  uint16_t *va = vbA + w * NT * kVTile, *vb = vbB + w * NT * kVTile;
  constexpr int KS = 64 * NT;  // keys per step
  const int spw = tpw / NT;     // steps per wave and chunk

  // Chunk i of this workgroup: unit u = c / P = row * nkv + kh, part = c % P, keys [part*CH, +CH).
  struct Chunk {
    int row, kh, part, lo, hi;  // hi: end of the chunk's keys (<= lo: none)
    rsrc_t kr, vr;
  };
  // A row's length and cache row are read one chunk ahead with ordinary vector loads (so they arrive
  // in order with the tile loads and never stall the pipeline); they are needed when the chunk's
  // first tile is requested. For the first chunk only the cache row is needed up front: its tiles
  // are requested over the whole cache row and keys past the length are masked when computed.
  struct Meta {
    int lraw, craw, praw, sraw;
  };
  auto ids = [&](int i, Chunk &k) {
    const int c = (int)blockIdx.x + i * G;
    const int u = c / P;
    k.part = c - u * P;
    k.row = u / nkv;
    k.kh = u - k.row * nkv;
    k.lo = k.part * CH;
  };
  const rsrc_t lens_r = make_rsrc(lens, (uint32_t)b * 4u);
  const rsrc_t map_r = make_rsrc(rowmap, rowmap ? (uint32_t)b * 4u : 0u);
  const rsrc_t pos_r = make_rsrc(si.pos, FUSED ? (uint32_t)b * 4u : 0u);
  const rsrc_t slot_r = make_rsrc(si.slot, FUSED ? (uint32_t)b * 4u : 0u);
  // The row map is requested first, and only when there is one: loads complete in issue order, so the
  // first tile (which needs only the cache row) then never waits for the lengths or positions.
  auto meta_load = [&](int i) {
    Meta m{0, 0, 0, 0};
    if (i < nmine) {
      Chunk k;
      ids(i, k);
      m.craw = k.row;
      if (rowmap) m.craw = bld4(map_r, (uint32_t)k.row * 4u);
      m.lraw = bld4(lens_r, (uint32_t)k.row * 4u);
      if (FUSED) {
        m.praw = bld4(pos_r, (uint32_t)k.row * 4u);
        m.sraw = bld4(slot_r, (uint32_t)k.row * 4u);
      }
    }
    return m;
  };
  auto resolve = [&](int i, const Meta &m, bool exact, Chunk &k) {
    ids(i, k);
    const int crow = __builtin_amdgcn_readfirstlane(m.craw);
    const bool ok = i < nmine && crow >= 0 && crow < cache_rows;
    const int64_t cb = (int64_t)(ok ? crow : 0) * s_kb + (int64_t)k.kh * s_kh;
    uint32_t bound = 0;
    k.hi = 0;
    if (ok) {
      if (exact) {
        const int L = min(max(__builtin_amdgcn_readfirstlane(m.lraw), 0), cache_len);
        k.hi = min(k.lo + CH, L);
        bound = k.hi > 0 ? (uint32_t)k.hi * row_bytes : 0u;
      } else {
        k.hi = k.lo + CH;  // refined by hi_of() before the chunk is computed
        bound = full_row;
      }
    }
    k.kr = make_rsrc_wave(kc + cb, bound);
    k.vr = make_rsrc_wave(vc + cb, bound);
  };
  auto hi_of = [&](const Chunk &k, const Meta &m, int i) {
    const int crow = __builtin_amdgcn_readfirstlane(m.craw);
    if (i >= nmine || crow < 0 || crow >= cache_rows) return 0;
    const int L = min(max(__builtin_amdgcn_readfirstlane(m.lraw), 0), cache_len);
    return min(k.lo + CH, L);
  };
  auto load_q = [&](const Chunk &k, int i, u32x4 &q0, u32x4 &q1) {
    // past the last chunk the row may not exist: an empty range, nothing is read
    const rsrc_t qr = make_rsrc(q + (int64_t)(i < nmine ? k.row : 0) * s_qb + (int64_t)k.kh * group * s_qh,
                                i < nmine ? (uint32_t)(group * s_qh * 2) : 0u);
    const uint32_t qo = (uint32_t)(tl.r16 * s_qh * 2) + 16u * tl.g;
    q0 = bld16(qr, qo);
    q1 = bld16(qr, qo + 64u);
  };
  // FUSED: one head per lane -- lanes r16 < group the q heads kh*group + r16, lane kLaneK the k head,
  // lane kLaneV the v head of the chunk's row -- and its partner chunks (dims 8g.., 32+8g..) of qkv and
  // bias, plus the position's cos / sin chunks, requested one chunk ahead like q; rows / positions that
  // do not exist read zeros.
  struct QkvRaw {
    u32x4 w[2], bb[2], cs[2], sn[2];
  };
  const int H = nq + 2 * nkv;
  auto lane_head = [&](const Chunk &k) {
    return tl.r16 < group ? k.kh * group + tl.r16
                          : tl.r16 == kLaneK ? nq + k.kh : tl.r16 == kLaneV ? nq + nkv + k.kh : 0;
  };
  auto load_qkv = [&](const Chunk &k, int i, const Meta &m, QkvRaw &r) {
    const bool live = i < nmine;
    const int p = __builtin_amdgcn_readfirstlane(m.praw);
    const bool pv = live && p >= 0 && p < si.n_tab;
    const rsrc_t xr = make_rsrc_wave(si.qkv + (int64_t)(live ? k.row : 0) * si.s_qkv, live ? (uint32_t)H * 128u : 0u);
    const rsrc_t br = make_rsrc(si.bias, si.bias ? (uint32_t)H * 128u : 0u);
    const rsrc_t cr = make_rsrc_wave(si.cos_tab + (int64_t)(pv ? p : 0) * si.s_cs, pv ? 128u : 0u);
    const rsrc_t sr = make_rsrc_wave(si.sin_tab + (int64_t)(pv ? p : 0) * si.s_cs, pv ? 128u : 0u);
    const uint32_t og = 16u * tl.g, ho = (uint32_t)lane_head(k) * 128u + og;
    r.w[0] = bld16(xr, ho);
    r.w[1] = bld16(xr, ho + 64u);
    r.bb[0] = bld16(br, ho);
    r.bb[1] = bld16(br, ho + 64u);
    r.cs[0] = bld16(cr, og);
    r.cs[1] = bld16(cr, og + 64u);
    r.sn[0] = bld16(sr, og);
    r.sn[1] = bld16(sr, og + 64u);
  };
  // FUSED, at a chunk's first step: one RoPE pass per lane gives q (lanes r16 < group: the Q^T operand),
  // the new k (lane kLaneK) and v (lane kLaneV: x narrowed, not rotated); the key column they replace
  // when the row attends the cache row it stores into; the unit's first chunk (wave 0) writes k / v to
  // the cache and q to qo, as k_bias_rope_store would.
  KVPatch pt;
  pt.col = -1;
  auto apply_qkv = [&](const Chunk &k, int i, const Meta &m, const QkvRaw &r, u32x4 &q0, u32x4 &q1) {
    const bool live = i < nmine;
    const int p = __builtin_amdgcn_readfirstlane(m.praw);
    const bool pv = live && p >= 0 && p < si.n_tab;
    const int crow = __builtin_amdgcn_readfirstlane(m.craw);
    const int srow = __builtin_amdgcn_readfirstlane(m.sraw);
    const int sidx = pv ? p % si.ring : 0;
    const bool store_ok = pv && srow >= 0 && srow < cache_rows && sidx < cache_len;
    float xl[8], xh[8], ol[8], oh[8];
    rope_x(r.w[0], r.w[1], r.bb[0], r.bb[1], si.bias != nullptr, xl, xh);
    rope_rotate_f(xl, xh, r.cs[0], r.cs[1], r.sn[0], r.sn[1], ol, oh);
    const bool vlane = tl.r16 == kLaneV;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ol[j] = vlane ? xl[j] : ol[j];
      oh[j] = vlane ? xh[j] : oh[j];
    }
    rope_narrow(ol, oh, pt.lo, pt.hi);
    const bool qlive = pv && tl.r16 < group;
    const u32x4 z{0u, 0u, 0u, 0u};
    q0 = qlive ? pt.lo : z;  // unknown position: the reference reads no table row; q is zero here
    q1 = qlive ? pt.hi : z;
    pt.col = (store_ok && srow == crow) ? sidx : -1;
    if (k.part == 0 && w == 0) {
      uint16_t *dst = nullptr;
      if (store_ok && (tl.r16 == kLaneK || vlane))
        dst = (vlane ? vc : kc) + (int64_t)srow * s_kb + (int64_t)k.kh * s_kh + (int64_t)sidx * s_ks;
      else if (si.qo && qlive)
        dst = si.qo + (int64_t)k.row * si.s_qo_r + (int64_t)(k.kh * group + tl.r16) * si.s_qo_h;
      if (dst) {
        st16(dst + 8 * tl.g, pt.lo);
        st16(dst + 32 + 8 * tl.g, pt.hi);
      }
    }
  };

  SoftmaxState S;
  S.reset();

  // End of chunk i: every wave parks its state in LDS and counts itself in; the last of the NW waves to
  // arrive merges the partials and writes the output (a row within one chunk) or the chunk's partial,
  // while the others go straight on to their next tiles. No wave waits for another here, so each keeps
  // its loads flowing (a barrier would hold every wave of the workgroup for the slowest one). Chunks
  // without keys are skipped by every wave alike, so the merge count n and its LDS buffer (n & 1) are
  // the same in every wave; before a wave parks merge n in a buffer it waits until that buffer's merge
  // n - 2 is complete (mseq), a wait that ends because a merging wave waits for nothing.
  int nfin = 0;
  auto finish_chunk = [&](const Chunk &k, int L) {
    const int peff = L > 0 ? (L + CH - 1) / CH : 1;  // chunks with keys (an empty row still writes 0/0)
    if (k.part >= peff) {  // no key of this row falls in this chunk
      S.reset();
      return;
    }
    const int n = nfin++;
    const int bsel = n & 1;
    float *mb = mrg[bsel], *lb = mb + NW * 16, *ob = mb + NW * 32;
    const float lsum = sum_over_groups(S.lsum);
    if (NW > 1) {
      while (lds_read_word(&mseq[bsel]) < n - 2) __builtin_amdgcn_s_sleep(1);
    }
    if (tl.g == 0) {
      mb[w * 16 + tl.r16] = S.m;
      lb[w * 16 + tl.r16] = lsum;
    }
    lds_store_4x16(ob + (w * 16 + tl.r16) * kOb + 4 * tl.g, S.o[0], S.o[1], S.o[2], S.o[3]);
    S.reset();
    if (NW > 1) {
      if (lds_add_word(&marr[bsel], 1) != NW - 1) return;
      lds_write_word(&marr[bsel], 0);  // the buffer's next arrivals come after mseq says n is merged
    } else {
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the parked state is readable
    }
    // one lane per (head, 4 dims): 16-byte reads of the parked O rows, one 8-byte store per lane
    for (int t = lane; t < group * 16; t += 64) {
      const int head = t >> 4, d4 = (t & 15) * 4;
      float mv[NW];
      float M = kNegInf;
#pragma unroll
      for (int v = 0; v < NW; ++v) {
        mv[v] = mb[v * 16 + head];
        M = fmaxf(M, mv[v]);
      }
      f32x4 num = {0.f, 0.f, 0.f, 0.f};
      float den = 0.f;
#pragma unroll
      for (int v = 0; v < NW; ++v) {
        const float wt = (mv[v] == kNegInf) ? 0.f : fast_exp2((mv[v] - M) * sl2);
        const f32x4 o = *reinterpret_cast<const f32x4 *>(ob + (v * 16 + head) * kOb + d4);
        num += wt * o;
        den += wt * lb[v * 16 + head];
      }
      const int hq = k.kh * group + head;
      if (peff == 1) {
        uint2 pk;
        pk.x = pack_bf16x2(num[0] / den, num[1] / den);
        pk.y = pack_bf16x2(num[2] / den, num[3] / den);
        *reinterpret_cast<uint2 *>(out + (int64_t)k.row * s_ob + (int64_t)hq * s_oh + d4) = pk;
      } else {
        const int64_t pi = ((int64_t)k.row * nq + hq) * P + k.part;
        *reinterpret_cast<f32x4 *>(acc_ws + pi * 64 + d4) = num;
        if (d4 == 0) {
          ml_ws[pi * 2] = M;
          ml_ws[pi * 2 + 1] = den;
        }
      }
    }
    if (NW > 1) lds_write_word(&mseq[bsel], n);  // after the reads above: the buffer may be reused
  };

  // The wave's step sequence: (chunk i, step j), i = 0..nmine-1, j = 0..spw-1, in two register
  // buffers with the loads always one tile ahead (past the end they read zeros, no memory traffic).
  Meta mcur = meta_load(0);
  Chunk cur, nxt;
  resolve(0, mcur, /*exact=*/false, cur);
  // the first tile goes out before anything that waits for the lengths or positions
  KTile A[NT], B[NT];
  load_step<NT>(A, va, cur.kr, cur.vr, (uint32_t)(cur.lo + KS * w), tl);
  Meta mnxt = meta_load(1);
  u32x4 qc0, qc1, qn0, qn1;
  QkvRaw rq;  // FUSED: raw qkv / bias / table chunks of the chunk about to start
  if (FUSED)
    load_qkv(cur, 0, mcur, rq);
  else
    load_q(cur, 0, qc0, qc1);
  int i = 0, j = 0;
  int hi = 0;
  bool fresh = true;  // cur's hi not refined yet
  // always inlined: each call site then sees which V buffer (vbA or vbB) it reads and writes
  auto step = [&](KTile (&X)[NT], uint16_t *xv, KTile (&Y)[NT], uint16_t *yv) __attribute__((always_inline)) -> bool {
    // request the tile after (i, j) into Y, then consume X
    const bool last_tile = (j + 1 == spw);
    Meta mnn{0, 0};
    if (last_tile) {
      resolve(i + 1, mnxt, /*exact=*/true, nxt);
      mnn = meta_load(i + 2);
      if (!FUSED) load_q(nxt, i + 1, qn0, qn1);
    }
    {
      // one load sequence for both cases (operands selected): with two, the compiler's wait
      // bookkeeping merges their states conservatively and drains every load in flight
      const rsrc_t kr = last_tile ? nxt.kr : cur.kr;
      const rsrc_t vr = last_tile ? nxt.vr : cur.vr;
      const int tn = last_tile ? nxt.lo + KS * w : cur.lo + KS * (w + NW * (j + 1));
      load_step<NT>(Y, yv, kr, vr, (uint32_t)tn, tl);
    }
    if (fresh) {
      hi = hi_of(cur, mcur, i);
      if (FUSED) apply_qkv(cur, i, mcur, rq, qc0, qc1);
      fresh = false;
    }
    const int t0 = cur.lo + KS * (w + NW * j);
    if (t0 < hi) compute_step<NT, 16 * NT, FUSED>(X, xv, t0, hi, qc0, qc1, sl2, S, tl, lane, &pt);
    if (FUSED && j == 0) {
      // the next chunk's qkv rows go out now, a whole chunk ahead of their use, into the registers this
      // chunk's rows were just consumed from (no copy at the transition): requested at the chunk's last
      // step they queued behind a step's worth of tile loads and held up every transition. Their
      // metadata arrived with the tile just computed.
      Chunk kn;
      ids(i + 1, kn);
      load_qkv(kn, i + 1, mnxt, rq);
    }
    if (last_tile) {
      const int L = (i < nmine) ? min(max(__builtin_amdgcn_readfirstlane(mcur.lraw), 0), cache_len) : 0;
      const int crow = __builtin_amdgcn_readfirstlane(mcur.craw);
      finish_chunk(cur, (crow < 0 || crow >= cache_rows) ? 0 : L);
      ++i;
      j = 0;
      cur = nxt;
      mcur = mnxt;
      mnxt = mnn;
      if (!FUSED) {
        qc0 = qn0;
        qc1 = qn1;
      }
      fresh = true;
      return i < nmine;
    }
    ++j;
    return true;
  };
  // the first step is peeled: it always takes chunk 0's q (or qkv) from the prologue's loads, so the
  // loop never sees those loads pending (otherwise registers they wrote, reused later, cost a full drain)
  if (step(A, va, B, vb)) {
    for (;;) {
      if (!step(B, vb, A, va)) break;
      if (!step(A, va, B, vb)) break;
    }
  }
  // the request past the last chunk still writes (zeros) into LDS: let it land before the wave ends.
  // s_waitcnt vmcnt(0).
  __builtin_amdgcn_s_waitcnt(0x0F70);
}

// Merges the chunks of rows longer than one chunk: one thread per (row, q head, dim); rows that fit one
// chunk were written by the streaming kernel and are skipped. All of a thread's partial loads are
// independent, so the kernel costs about one memory round trip.
__global__ __launch_bounds__(256) void k_decode_stream_combine(
    const float *__restrict__ acc_ws, const float *__restrict__ ml_ws, const int32_t *__restrict__ lens,
    const int32_t *__restrict__ rowmap, uint16_t *__restrict__ out, int64_t s_ob, int64_t s_oh, int b, int nq,
    int cache_rows, int cache_len, int CH, int P, float sl2) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)b * nq * 64) return;
  const int d = (int)(t & 63);
  const int pair = (int)(t >> 6);
  const int row = pair / nq, h = pair - row * nq;
  const int crow = rowmap ? rowmap[row] : row;
  int L = lens[row];
  L = (crow < 0 || crow >= cache_rows) ? 0 : min(max(L, 0), cache_len);
  const int peff = L > 0 ? (L + CH - 1) / CH : 1;
  if (peff == 1) return;
  const float *ml = ml_ws + (int64_t)pair * P * 2;
  const float *acc = acc_ws + (int64_t)pair * P * 64 + d;
  float M = kNegInf;
  for (int pp = 0; pp < peff; ++pp) M = fmaxf(M, ml[2 * pp]);
  float num = 0.f, den = 0.f;
  for (int pp = 0; pp < peff; ++pp) {
    const float mv = ml[2 * pp];
    const float wt = (mv == kNegInf) ? 0.f : fast_exp2((mv - M) * sl2);
    num += wt * acc[pp * 64];
    den += wt * ml[2 * pp + 1];
  }
  out[(int64_t)row * s_ob + (int64_t)h * s_oh + d] = (uint16_t)(pack_bf16x2(num / den, 0.f) & 0xffffu);
}

template <int NW, int NT, bool FUSED>
static void launch_stream(int grid, hipStream_t st, const uint16_t *q, int64_t s_qb, int64_t s_qh, uint16_t *kc,
                          uint16_t *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks, int cache_rows, int cache_len,
                          const int32_t *lens, const int32_t *rowmap, uint16_t *out, int64_t s_ob, int64_t s_oh,
                          float *acc_ws, float *ml_ws, int b, int nq, int nkv, int group, int tpw, int P, float sl2,
                          const StoreIn &si) {
  auto kern = k_decode_stream<NW, NT, FUSED>;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * NW), 0, st, q, s_qb, s_qh, kc, vc, s_kb, s_kh, s_ks, cache_rows,
                     cache_len, lens, rowmap, out, s_ob, s_oh, acc_ws, ml_ws, b, nq, nkv, group, tpw, P, sl2, si);
}

static inline bool al16s(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// decode_rows.hip
bool rows_launch(int grid, hipStream_t st, const uint16_t *q, int64_t s_qb, int64_t s_qh, uint16_t *kc, uint16_t *vc,
                 int64_t s_kb, int64_t s_kh, int cache_rows, int cache_len, const int32_t *lens, const int32_t *rowmap,
                 uint16_t *out, int64_t s_ob, int64_t s_oh, int b, int nq, int nkv, int group, float sl2,
                 const StoreIn &si);

// Body of a8_decode_attn_stream and a8_store_decode_stream (fused = si.qkv != nullptr: q is unused, the
// store's inputs are in si). Checks the decode arguments, launches the streaming kernel and,
// for rows longer than a chunk, the merge kernel.
static int stream_entry(const char *fn, const void *q, int64_t s_qb, int64_t s_qh, void *kc, void *vc,
                        int64_t s_kb, int64_t s_kh, int64_t s_ks, int cache_rows, int cache_len,
                        const int32_t *lens, const int32_t *rowmap, void *out, int64_t s_ob, int64_t s_oh,
                        float *acc_ws, float *ml_ws, int64_t ws_row_splits, int b, int nq, int nkv, int hd,
                        int waves, int tiles_per_wave, int grid, float scale, int phases, const StoreIn &si,
                        void *stream) {
  const bool fused = si.qkv != nullptr;
  if (hd != 64 && (fused || hd != 128))
    return set_error(A8_EUNSUP, "%s: head_dim %d not supported (64; 128 through the unfused call)", fn, hd);
  if (b < 0 || nq <= 0 || nkv <= 0 || nq % nkv || cache_rows < 0 || cache_len < 0)
    return set_error(A8_EINVAL, "%s: bad sizes b=%d nq=%d nkv=%d", fn, b, nq, nkv);
  const int group = nq / nkv;
  if (group > 16) return set_error(A8_EUNSUP, "%s: GQA group %d > 16 not supported", fn, group);
  if (waves != 1 && waves != 2 && waves != 4 && waves != 8)
    return set_error(A8_EINVAL, "%s: waves must be 1, 2, 4 or 8 (got %d)", fn, waves);
  if (waves == 8)  // 8 waves' double-buffered V tiles and merge buffers exceed the 160 KB of LDS
    return set_error(A8_EUNSUP, "%s: 8 waves per workgroup not supported (1, 2 or 4)", fn);
  if (tiles_per_wave < 1 || tiles_per_wave > 64 || grid < 1)
    return set_error(A8_EINVAL, "%s: tiles_per_wave %d / grid %d out of range", fn, tiles_per_wave, grid);
  if (b == 0) return 0;
  if ((!fused && !q) || !kc || !vc || !lens || !out) return set_error(A8_EINVAL, "%s: null pointer", fn);
  const int CH = waves * tiles_per_wave * 64;
  const int P = cache_len > 0 ? (cache_len + CH - 1) / CH : 1;
  const int64_t NC = (int64_t)b * nkv * P;
  if (NC > (1ll << 30)) return set_error(A8_EINVAL, "%s: too many chunks", fn);
  if (P > 1 && (!acc_ws || !ml_ws || (int64_t)b * P > ws_row_splits))
    return set_error(A8_EWSPACE, "%s: workspace holds %lld row-splits, need b*%d = %lld", fn,
                     (long long)ws_row_splits, P, (long long)b * P);
  if (s_ks != hd)
    return set_error(A8_EUNSUP, "%s: cache positions must be contiguous rows (s_ks %lld)", fn, (long long)s_ks);
  if ((!fused && !al16s(q)) || !al16s(kc) || !al16s(vc) || !al16s(out) || (P > 1 && !al16s(acc_ws)) ||
      ((fused ? 0 : (s_qb | s_qh)) | s_kb | s_kh | s_ks | s_ob | s_oh) & 7)
    return set_error(A8_EALIGN, "%s: pointers must be 16-byte aligned and strides multiples of 8", fn);
  if (hd != 64)  // the generic-head kernel (one launch, no workspace)
    return attn_cols_decode(fn, q, s_qb, s_qh, kc, vc, s_kb, s_kh, cache_rows, cache_len, lens, rowmap, out, s_ob,
                            s_oh, b, nq, nkv, hd, scale, (hipStream_t)stream);
  if (grid > NC) grid = (int)NC;
  const hipStream_t st = (hipStream_t)stream;
  const float sl2 = scale * kLog2e;
  const auto *qq = (const uint16_t *)q;
  auto *kk = (uint16_t *)kc;
  auto *vv = (uint16_t *)vc;
  auto *oo = (uint16_t *)out;
  // whole rows per workgroup at 4 waves x one tile per step (the peak-load shape): k_decode_rows, same
  // results bit for bit; phases bit 2 keeps k_decode_stream (for timing the two apart)
  const bool rows = (phases & 1) && P == 1 && waves == 4 && !(phases & 4) &&
                    rows_launch(grid, st, qq, s_qb, s_qh, kk, vv, s_kb, s_kh, cache_rows, cache_len, lens, rowmap, oo,
                                s_ob, s_oh, b, nq, nkv, group, sl2, si);
  if (rows) return (int)hipGetLastError();
  if (phases & 1) {
#define A8_STREAM_ARGS grid, st, qq, s_qb, s_qh, kk, vv, s_kb, s_kh, s_ks, cache_rows, cache_len, lens, rowmap, oo, \
                       s_ob, s_oh, acc_ws, ml_ws, b, nq, nkv, group, tiles_per_wave, P, sl2, si
    // two-tile steps where the tile count allows and the LDS holds them (4 waves x 2 x 2 V tiles and
    // the merge buffers do not fit in 160 KB)
    const bool nt2 = (tiles_per_wave % 2 == 0) && waves <= 2;
    switch ((waves * 2 + (nt2 ? 1 : 0)) * 2 + (fused ? 1 : 0)) {
      case 4: launch_stream<1, 1, false>(A8_STREAM_ARGS); break;
      case 5: launch_stream<1, 1, true>(A8_STREAM_ARGS); break;
      case 6: launch_stream<1, 2, false>(A8_STREAM_ARGS); break;
      case 7: launch_stream<1, 2, true>(A8_STREAM_ARGS); break;
      case 8: launch_stream<2, 1, false>(A8_STREAM_ARGS); break;
      case 9: launch_stream<2, 1, true>(A8_STREAM_ARGS); break;
      case 10: launch_stream<2, 2, false>(A8_STREAM_ARGS); break;
      case 11: launch_stream<2, 2, true>(A8_STREAM_ARGS); break;
      case 17: launch_stream<4, 1, true>(A8_STREAM_ARGS); break;
      default: launch_stream<4, 1, false>(A8_STREAM_ARGS); break;
    }
#undef A8_STREAM_ARGS
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  if ((phases & 2) && P > 1) {
    const unsigned cgrid = (unsigned)(((int64_t)b * nq * 64 + 255) / 256);
    hipLaunchKernelGGL(k_decode_stream_combine, dim3(cgrid), dim3(256), 0, st, acc_ws, ml_ws, lens, rowmap, oo,
                       s_ob, s_oh, b, nq, cache_rows, cache_len, CH, P, sl2);
    return (int)hipGetLastError();
  }
  return 0;
}

}  // namespace a8

extern "C" int a8_decode_attn_stream(const void *q, int64_t s_qb, int64_t s_qh,
                                     const void *kc, const void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                                     int cache_rows, int cache_len,
                                     const int32_t *lens, const int32_t *rowmap,
                                     void *out, int64_t s_ob, int64_t s_oh,
                                     float *acc_ws, float *ml_ws, int64_t ws_row_splits,
                                     int b, int nq, int nkv, int hd, int waves, int tiles_per_wave, int grid,
                                     float scale, int phases, void *stream) {
  using namespace a8;
  const StoreIn none{};
  return stream_entry("decode_attn_stream", q, s_qb, s_qh, const_cast<void *>(kc), const_cast<void *>(vc), s_kb,
                      s_kh, s_ks, cache_rows, cache_len, lens, rowmap, out, s_ob, s_oh, acc_ws, ml_ws,
                      ws_row_splits, b, nq, nkv, hd, waves, tiles_per_wave, grid, scale, phases, none, stream);
}

extern "C" int a8_store_decode_stream(const void *qkv, int64_t s_qkv, const void *bias,
                                      const void *cos_tab, const void *sin_tab, int64_t s_cs, int n_tab,
                                      const int32_t *pos, const int32_t *slot,
                                      void *qo, int64_t s_qo_r, int64_t s_qo_h,
                                      void *kc, void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                                      int cache_rows, int cache_len, const int32_t *lens,
                                      const int32_t *rowmap, void *out, int64_t s_ob, int64_t s_oh,
                                      float *acc_ws, float *ml_ws, int64_t ws_row_splits,
                                      int b, int nq, int nkv, int hd, int ring, int waves, int tiles_per_wave,
                                      int grid, float scale, int phases, void *stream) {
  using namespace a8;
  if (ring <= 0 || n_tab < 0) return set_error(A8_EINVAL, "store_decode_stream: bad ring %d / n_tab %d", ring, n_tab);
  if (b > 0 && (!qkv || !cos_tab || !sin_tab || !pos || !slot))
    return set_error(A8_EINVAL, "store_decode_stream: null pointer");
  if (b > 0 && (!al16s(qkv) || !al16s(cos_tab) || !al16s(sin_tab) || (bias && !al16s(bias)) || (qo && !al16s(qo)) ||
                (s_qkv | s_cs | (qo ? (s_qo_r | s_qo_h) : 0)) & 7))
    return set_error(A8_EALIGN, "store_decode_stream: pointers must be 16-byte aligned and strides multiples of 8");
  if (nkv > 0 && nq / nkv > kLaneK)  // lanes kLaneK / kLaneV compute k / v next to the q heads
    return set_error(A8_EUNSUP, "store_decode_stream: GQA group %d > %d not supported", nq / nkv, kLaneK);
  if (b > 0 && (phases & 1) == 0)  // the store is part of the streaming kernel
    return set_error(A8_EINVAL, "store_decode_stream: phases must include the streaming kernel (bit 0)");
  StoreIn si{};
  si.slot = slot;
  si.qkv = (const uint16_t *)qkv;
  si.s_qkv = s_qkv;
  si.bias = (const uint16_t *)bias;
  si.cos_tab = (const uint16_t *)cos_tab;
  si.sin_tab = (const uint16_t *)sin_tab;
  si.s_cs = s_cs;
  si.n_tab = n_tab;
  si.pos = pos;
  si.qo = (uint16_t *)qo;
  si.s_qo_r = s_qo_r;
  si.s_qo_h = s_qo_h;
  si.ring = ring;
  if (b == 0) return 0;
  return stream_entry("store_decode_stream", nullptr, 0, 0, kc, vc, s_kb, s_kh, s_ks, cache_rows, cache_len, lens,
                      rowmap, out, s_ob, s_oh, acc_ws, ml_ws, ws_row_splits, b, nq, nkv, hd, waves, tiles_per_wave,
                      grid, scale, phases, si, stream);
}

// Launch shape of a8_decode_attn_stream. Whole rows of at most 32 tiles (the slow stack's 2048-position cache)
// whose units (row, kv head) reach half the compute units take one workgroup of 4 waves per unit while the units
// fit the compute units (k_decode_unit: every unit streams at once), else two units per workgroup up to twice the
// compute units (k_decode_rows). Measured on MI355X at KV 2048, fused store + decode, us per layer: 128 units
// (64 rows) 16.6 one per workgroup against 17.9 for the split kernel; 256 units 24.9 against 30.9 for two per
// workgroup on 128; 288 units 31.5 two per workgroup against 35.9 one per workgroup (32 compute units then
// hold two); 384 units (C3) 36.2-36.6 two per workgroup against 39.0 one per workgroup. Beyond that, and for
// other row lengths: a workgroup target of 3/4 of the compute units, chunks per unit only as many as needed to
// reach it (long rows of few units), and a grid that divides the chunk count evenly. The workspace caps the
// chunk count per unit.
extern "C" int a8_decode_choose_stream(int b, int nkv, int cache_len, int64_t cap_row_splits, int n_cu,
                                       int *waves_out, int *tpw_out, int *grid_out) {
  using namespace a8;
  if (b < 1 || nkv < 1 || cache_len < 0 || n_cu < 1 || !waves_out || !tpw_out || !grid_out)
    return set_error(A8_EINVAL, "decode_choose_stream: bad arguments b=%d nkv=%d n_cu=%d", b, nkv, n_cu);
  const int64_t tiles = cache_len > 0 ? (cache_len + 63) / 64 : 1;
  const int nw = tiles >= 8 ? 4 : tiles >= 4 ? 2 : 1;
  const int64_t units = (int64_t)b * nkv;
  if (nw == 4 && tiles <= 32 && 2 * units >= n_cu && units <= 2 * (int64_t)n_cu) {
    *waves_out = 4;
    *tpw_out = (int)((tiles + 3) / 4);
    *grid_out = (int)(units <= n_cu ? units : (units + 1) / 2);
    return 0;
  }
  const int64_t g0 = n_cu * 3 / 4 > 0 ? n_cu * 3 / 4 : 1;
  const int64_t p_want = (g0 + units - 1) / units;
  int64_t tpw = (tiles + nw * p_want - 1) / (nw * p_want);
  if (tpw < 1) tpw = 1;
  if (tpw > 64) tpw = 64;
  // chunk count per unit: at most what the workspace holds
  const int64_t pmax = cap_row_splits >= b ? cap_row_splits / b : 1;
  while (tpw < 64) {
    const int64_t P = (tiles + nw * tpw - 1) / (nw * tpw);
    if (P <= 1 || P <= pmax) break;
    tpw *= 2;
  }
  if (tpw > 64) tpw = 64;
  const int64_t P = (tiles + nw * tpw - 1) / (nw * tpw);
  const int64_t NC = units * P;
  const int64_t per = (NC + g0 - 1) / g0;  // chunks per workgroup
  const int64_t grid = (NC + per - 1) / per;
  *waves_out = nw;
  *tpw_out = (int)tpw;
  *grid_out = (int)grid;
  return 0;
}
