/*
 * a8attn.h -- C ABI of the MI355X (gfx950) attention hot path of the Audio8 streaming TTS engine.
 *
 * Three operators, each a drop-in for one function of the reference's operator module
 * (serve/fast_kernels.py of lvt1693/audio8-turbo-engine):
 *
 *   a8_bias_rope_store   fused qkv bias + rotate_half RoPE + K/V store into the slot cache
 *   a8_decode_attn       split-K flash-decoding over the slot cache (GQA), split + combine
 *   a8_prefill_attn      packed variable-length causal prefill attention over cache rows
 *
 * and the admission copy of a cached voice prefix's K/V into slots (a8_prefix_copy, an index-put of
 * serve/fast_engine.py), plus the launch-shape choosers and fused / alternative schedules below.
 *
 * Conventions shared by every entry point:
 *   - All tensors are bf16 (stored as 16-bit words) unless the argument says otherwise; index
 *     tensors are int32. Every pointer is a device pointer (hipMalloc'ed or a view into one).
 *   - Strides are in ELEMENTS, as torch reports them. The last (head_dim) axis is contiguous.
 *   - The slot cache is [cache_rows, nkv, cache_len, hd] with strides (s_kb, s_kh, s_ks, 1); K and
 *     V caches share strides (the reference kernels address both with the K strides). Row strides
 *     may be non-dense (the codec's byte-arena views).
 *   - Vector loads are 16 bytes wide: base pointers must be 16-byte aligned and every stride a
 *     multiple of 8 elements. Violations return A8_EALIGN without launching anything.
 *   - `stream` is a hipStream_t (torch.cuda.current_stream().cuda_stream). Entry points only
 *     enqueue work: no allocation, no synchronisation, so they are safe under stream capture.
 *   - Return value: 0 on success, a negative A8_E* code for a rejected argument (nothing launched;
 *     a8_last_error() has the message), or a positive hipError_t from the launch.
 *   - Device-side index data the host cannot see (pos, slot, lens, rowmap, plan entries) is
 *     bounds-checked in the kernels: a row whose slot / cache row lies outside [0, cache_rows),
 *     or whose position lies outside the cos/sin table or the cache, writes nothing instead of
 *     writing out of bounds (the reference leaves those cases undefined).
 */
#ifndef A8ATTN_H
#define A8ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define A8_EINVAL  (-1) /* shape / count argument out of range */
#define A8_EALIGN  (-2) /* pointer or stride not 16-byte aligned */
#define A8_EUNSUP  (-3) /* configuration this build does not implement (e.g. head_dim 96) */
#define A8_EWSPACE (-4) /* decode workspace too small for b * nsplit row-splits */

/* Library version string, "a8attn <version> gfx950 src:<hash>", the hash being that of the sources the library
 * was built from (so a stale build can be detected). No reference counterpart. */
const char *a8_version(void);

/* Message for the last negative status returned on the calling thread ("" if none). */
const char *a8_last_error(void);

/* File name of the HIP runtime this library is bound to (dladdr of hipLaunchKernel). Lets a
 * Python host check that it shares torch's runtime (same soname, loaded once). */
const char *a8_hip_runtime_path(void);

/*
 * Fused qkv bias + rotate_half RoPE + K/V store.
 * Replaces serve/fast_kernels.py:179-187 (bias_rope_store) and its kernel
 * _bias_rope_store_kernel (fast_kernels.py:139-176).
 *
 * qkv     [R, (nq + 2*nkv) * hd] row stride s_qkv; columns contiguous
 * bias    [(nq + 2*nkv) * hd] or NULL
 * cos_tab, sin_tab [n_tab, hd] row stride s_cs (rotate_half tables, see a1 _rope_tables)
 * pos, slot [R] int32
 * qo      [R, nq, hd] strides (s_qo_r, s_qo_h, 1)            <- rotated q; or NULL: no q (only the
 *                                                               k / v heads run; for a8_prefill_attn_qkv,
 *                                                               which forms q from qkv itself)
 * kc, vc  slot cache                                         <- rotated k / biased v at
 *                                                               [slot[r], h, pos[r] % ring, :]
 * Per row r and head h: x = f32(qkv) + f32(bias); q/k: o = bf16(x*cos + sign*x[(d+hd/2)%hd]*sin)
 * with sign = -1 for d < hd/2, evaluated without fused multiply-add; v: bf16(x).
 * hd: a multiple of 16 up to 256 (the engine's 64, and 128).
 */
int a8_bias_rope_store(const void *qkv, int64_t s_qkv, const void *bias,
                       const void *cos_tab, const void *sin_tab, int64_t s_cs, int n_tab,
                       const int32_t *pos, const int32_t *slot, int R,
                       void *qo, int64_t s_qo_r, int64_t s_qo_h,
                       void *kc, void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                       int cache_rows, int cache_len,
                       int nq, int nkv, int hd, int ring, void *stream);

/*
 * Split-K flash-decoding, GQA (group = nq / nkv <= 16), one query token per row.
 * Replaces serve/fast_kernels.py:271-290 (DecodeAttention.__call__) with its kernels
 * _dec_attn_split_kernel (193-235) and _dec_attn_combine_kernel (238-253).
 *
 * q       [b, nq, hd] strides (s_qb, s_qh, 1)
 * kc, vc  slot cache; query row i reads cache row rowmap[i] (i when rowmap == NULL)
 * lens    [b] int32: keys [0, lens[i]) are attended
 * out     [b, nq, hd] strides (s_ob, s_oh, 1)
 * acc_ws  fp32 workspace, >= ws_row_splits * nq * hd floats (DecodeAttention.acc_flat)
 * ml_ws   fp32 workspace, >= ws_row_splits * nq * 2 floats  (DecodeAttention.ml_flat)
 * counters  NULL, or int32 [>= b * nkv] that start at 0 (DecodeAttention.counters; every launch leaves
 *         them at 0): with counters the split kernel merges the splits itself -- the last split
 *         workgroup of each (row, kv head) to finish combines the row's partials with the combine
 *         kernel's arithmetic -- and no combine launch follows (one launch instead of two). Calls that
 *         share counters or the workspace must not overlap in time (one stream).
 * nsplit  key-range splits per row (>= 1; b * nsplit <= ws_row_splits). With nsplit == 1 the
 *         split kernel writes `out` directly and no combine runs.
 * waves   wavefronts per workgroup that share one split's key range: 1, 2, 4 or 8.
 * phases  bit 0: run the split kernel, bit 1: run the combine kernel (3 = both; the normal value).
 *         Running them separately lets a caller time each kernel. With counters, bit 1 is ignored.
 * Rows with lens == 0 produce NaN (0/0), exactly as the reference's combine does.
 * The cache positions must be contiguous rows (s_ks == hd, true of every reference cache view);
 * otherwise A8_EUNSUP. hd: 64, or 128 (the generic-head kernel: one launch whatever nsplit / waves, the
 * workspace and counters unused; same results up to fp32 rounding). The decode entry points below
 * (_stream, _flat, _noalloc) take hd 128 the same way; the fused store + decode ones (a8_store_decode_*)
 * take 64 only (a caller with hd 128 calls a8_bias_rope_store, then the decode).
 */
int a8_decode_attn(const void *q, int64_t s_qb, int64_t s_qh,
                   const void *kc, const void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                   int cache_rows, int cache_len,
                   const int32_t *lens, const int32_t *rowmap,
                   void *out, int64_t s_ob, int64_t s_oh,
                   float *acc_ws, float *ml_ws, int64_t ws_row_splits,
                   int32_t *counters, int64_t n_counters,
                   int b, int nq, int nkv, int hd, int nsplit, int waves, float scale,
                   int phases, void *stream);

/*
 * a8_decode_attn without a caller workspace, for callers that cannot allocate device memory (code
 * being captured into a HIP graph, tight serving loops, harnesses that forbid hipMalloc). No counterpart
 * in the reference: its DecodeAttention always owns a workspace (fast_kernels.py:256-269).
 * Same arguments, kernels and results (bit for bit) as a8_decode_attn with counters == NULL and
 * phases == 3; the split partials go to a fixed device array of A8_NOALLOC_SCRATCH_BYTES that the library
 * holds on each GPU until the process ends; the array used is the one on the device `stream` belongs to
 * (the current device for the null stream), looked up on that device's first call, which is best made
 * outside graph capture. Allocates nothing. nsplit > 1 with hd 64 needs
 * b * nq * nsplit * (hd + 2) * 4 <= A8_NOALLOC_SCRATCH_BYTES, else A8_EWSPACE (hd 128 uses no partials).
 * Every call on one GPU shares that GPU's array: calls that overlap in time on one GPU (two streams, two
 * host threads) race; serialise them.
 */
#define A8_NOALLOC_SCRATCH_BYTES (8ll << 20)
int a8_decode_attn_noalloc(const void *q, int64_t s_qb, int64_t s_qh,
                           const void *kc, const void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                           int cache_rows, int cache_len,
                           const int32_t *lens, const int32_t *rowmap,
                           void *out, int64_t s_ob, int64_t s_oh,
                           int b, int nq, int nkv, int hd, int nsplit, int waves, float scale,
                           void *stream);

/*
 * Launch-shape policy for a8_decode_attn on this GPU: picks (nsplit, waves) so that
 * b * nkv * nsplit workgroups fill n_cu compute units for keys up to cache_len.
 * nsplit_req is the caller's request (the reference's per-bucket heuristic, fast_engine.py:776):
 * the result is never below it. The result respects nsplit_max and b * nsplit <= cap_row_splits.
 * Replaces the nsplit heuristic of serve/fast_engine.py:776, re-derived for 256 CUs.
 */
int a8_decode_choose(int b, int nkv, int cache_len, int nsplit_req, int nsplit_max,
                     int64_t cap_row_splits, int n_cu, int *nsplit_out, int *waves_out);

/*
 * Split-K flash-decoding, streaming schedule: the default decode launch. Same inputs, outputs and
 * semantics as a8_decode_attn (serve/fast_kernels.py:271-290 with the kernels 193-253). Each
 * (row, kv head) is cut into chunks of waves * tiles_per_wave * 64 keys, P = ceil(cache_len / chunk)
 * per row; `grid` persistent workgroups sweep the chunks in cache address order. Rows whose keys fit
 * in one chunk are written by that kernel; longer rows leave per-chunk partials in acc_ws / ml_ws
 * (b * P row-splits <= ws_row_splits) that a second, small kernel merges.
 * waves   1, 2, 4 or 8; tiles_per_wave >= 1; grid >= 1 (clamped to the chunk count).
 * phases  bit 0: streaming kernel, bit 1: merge kernel (3 = both; the normal value).
 * Use a8_decode_choose_stream for the launch shape.
 */
int a8_decode_attn_stream(const void *q, int64_t s_qb, int64_t s_qh,
                          const void *kc, const void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                          int cache_rows, int cache_len,
                          const int32_t *lens, const int32_t *rowmap,
                          void *out, int64_t s_ob, int64_t s_oh,
                          float *acc_ws, float *ml_ws, int64_t ws_row_splits,
                          int b, int nq, int nkv, int hd, int waves, int tiles_per_wave, int grid,
                          float scale, int phases, void *stream);

/*
 * Launch shape of a8_decode_attn_stream for b rows over a cache of cache_len positions on a GPU of
 * n_cu compute units, within a workspace of cap_row_splits row-splits. Replaces the per-bucket split
 * heuristic of serve/fast_engine.py:776 (tuned there for an 84-SM GPU).
 */
int a8_decode_choose_stream(int b, int nkv, int cache_len, int64_t cap_row_splits, int n_cu,
                            int *waves_out, int *tiles_per_wave_out, int *grid_out);

/*
 * a8_bias_rope_store followed by a8_decode_attn (serve/fast_engine.py:127-132) with the store done by
 * the split kernel: two launches (split, combine) instead of three, with the contract of
 * a8_store_decode_stream (same results bit for bit as the two calls at the same nsplit / waves, provided
 * no row attends a cache row that another row of the call stores into). phases must include bit 0.
 */
int a8_store_decode_split(const void *qkv, int64_t s_qkv, const void *bias,
                          const void *cos_tab, const void *sin_tab, int64_t s_cs, int n_tab,
                          const int32_t *pos, const int32_t *slot,
                          void *qo, int64_t s_qo_r, int64_t s_qo_h,
                          void *kc, void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                          int cache_rows, int cache_len, const int32_t *lens, const int32_t *rowmap,
                          void *out, int64_t s_ob, int64_t s_oh,
                          float *acc_ws, float *ml_ws, int64_t ws_row_splits,
                          int32_t *counters, int64_t n_counters,
                          int b, int nq, int nkv, int hd, int ring, int nsplit, int waves, float scale,
                          int phases, void *stream);

/*
 * Split-K flash-decoding in one launch for any mix of row lengths (replaces the split + combine pair of
 * serve/fast_kernels.py:193-253 behind DecodeAttention.__call__, 271-290). Same inputs, outputs and
 * semantics as a8_decode_attn. The kernel reads lens / rowmap, splits the (row, kv head) 64-key tiles
 * evenly over grid * 4 wavefronts, and merges rows that span several wavefronts inside the launch: the
 * last wavefront to finish a row (counted with an atomic in counters[row * nkv + kv head]) merges its
 * partials, in a fixed order, from acc_ws / ml_ws.
 * counters    int32 [n_counters >= b * nkv], all zero before the first call; every call leaves them
 *             zero. Shared by the calls of one workspace: calls that overlap on the GPU race.
 * acc_ws ...  2 * grid * 4 partial slots of (nq / nkv) x 64 floats: grid * 8 <= ws_row_splits * nkv.
 * b <= 2048 rows per call; grid from a8_decode_choose_flat.
 */
int a8_decode_attn_flat(const void *q, int64_t s_qb, int64_t s_qh,
                        const void *kc, const void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                        int cache_rows, int cache_len, const int32_t *lens, const int32_t *rowmap,
                        void *out, int64_t s_ob, int64_t s_oh,
                        float *acc_ws, float *ml_ws, int64_t ws_row_splits,
                        int32_t *counters, int64_t n_counters,
                        int b, int nq, int nkv, int hd, int grid, float scale, void *stream);

/*
 * a8_decode_attn_f32q replaces the PREC = "ieee" branch of serve/fast_kernels.py:271-290 (DecodeAttention
 * with an fp32 query, 279; kernels 193-253): q fp32 [b, nq, hd] (strides s_qb, s_qh), the caches and lens /
 * rowmap as a8_decode_attn; fp32 products q . k (k widened exactly), the softmax weights rounded to bf16 for
 * P.V, fp32 sums; out [b, nq, hd] bf16 (out_f32 = 0) or fp32 (out_f32 = 1), strides s_ob, s_oh. One launch,
 * no workspace; hd 64 or 128, at most 16 q heads per kv head.
 */
int a8_decode_attn_f32q(const float *q, int64_t s_qb, int64_t s_qh, const void *kc, const void *vc, int64_t s_kb,
                        int64_t s_kh, int64_t s_ks, int cache_rows, int cache_len, const int32_t *lens,
                        const int32_t *rowmap, void *out, int64_t s_ob, int64_t s_oh, int out_f32, int b, int nq,
                        int nkv, int hd, float scale, void *stream);

/*
 * Launch shape of a8_decode_attn_flat / a8_store_decode_flat (replaces the split heuristic of
 * serve/fast_engine.py:776): workgroups for b rows over a cache of cache_len positions on n_cu compute
 * units, within a workspace of cap_row_splits row-splits.
 */
int a8_decode_choose_flat(int b, int nkv, int cache_len, int64_t cap_row_splits, int n_cu, int *grid_out);

/*
 * a8_bias_rope_store followed by a8_decode_attn_flat (serve/fast_engine.py:127-132) in one launch, with
 * the contract of a8_store_decode_stream: same results bit for bit as the two calls, provided no row
 * attends a cache row that another row of the call stores into.
 */
int a8_store_decode_flat(const void *qkv, int64_t s_qkv, const void *bias,
                         const void *cos_tab, const void *sin_tab, int64_t s_cs, int n_tab,
                         const int32_t *pos, const int32_t *slot,
                         void *qo, int64_t s_qo_r, int64_t s_qo_h,
                         void *kc, void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                         int cache_rows, int cache_len, const int32_t *lens, const int32_t *rowmap,
                         void *out, int64_t s_ob, int64_t s_oh,
                         float *acc_ws, float *ml_ws, int64_t ws_row_splits,
                         int32_t *counters, int64_t n_counters,
                         int b, int nq, int nkv, int hd, int ring, int grid, float scale, void *stream);

/*
 * The decode tick's per-layer pair in one launch (serve/fast_engine.py:127-132: bias_rope_store, then
 * DecodeAttention). Same results as a8_bias_rope_store(qkv, ..., pos, slot, R = b, qo, kc, vc, ...)
 * followed by a8_decode_attn_stream(qo, ..., lens, rowmap, ...) at the same launch shape, bit for bit,
 * provided no row attends a cache row that another row of the call stores into (true for the engine's
 * tick: slot = row, rowmap NULL, fast_engine.py:752-753; and for distinct slots with rowmap = slot).
 * The streaming kernel computes each row's q and new k / v from qkv + bias + RoPE with the store
 * kernel's arithmetic, writes k / v to kc / vc[slot, :, pos % ring] and q to qo (skipped when qo is
 * NULL), and, when the row attends the cache row it stores into, takes the new key column from
 * registers. A row whose pos is outside [0, n_tab) stores nothing and attends with q = 0.
 * rowmap  cache row attended by query row r: rowmap[r], or r when NULL (as in a8_decode_attn_stream).
 * Other arguments: those of a8_bias_rope_store and a8_decode_attn_stream; phases must include bit 0.
 */
int a8_store_decode_stream(const void *qkv, int64_t s_qkv, const void *bias,
                           const void *cos_tab, const void *sin_tab, int64_t s_cs, int n_tab,
                           const int32_t *pos, const int32_t *slot,
                           void *qo, int64_t s_qo_r, int64_t s_qo_h,
                           void *kc, void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                           int cache_rows, int cache_len, const int32_t *lens, const int32_t *rowmap,
                           void *out, int64_t s_ob, int64_t s_oh,
                           float *acc_ws, float *ml_ws, int64_t ws_row_splits,
                           int b, int nq, int nkv, int hd, int ring, int waves, int tiles_per_wave,
                           int grid, float scale, int phases, void *stream);

/*
 * Packed causal prefill attention over keys already stored in cache rows.
 * Replaces serve/fast_kernels.py:350-358 (prefill_attention) and its kernel
 * _prefill_attn_kernel (296-332); the block plan is the reference's PrefillPlan
 * (fast_kernels.py:335-347) or the graph-mode plan of fast_engine.py:820-853.
 *
 * q, out  [R, nq, hd] packed rows, strides (s_qr, s_qh, 1) / (s_or, s_oh, 1)
 * kc, vc  slot cache
 * bq0, bn, bslot, bpos0 [nblk] int32: block j covers packed rows [bq0, bq0 + bn) (bn <= bm) at
 *         positions [bpos0, bpos0 + bn) of cache row bslot; keys [0, bpos0 + bn) are attended with
 *         key <= query position. Blocks with bn <= 0 are no-ops (graph-mode padding).
 * group   q heads per kv head (nq / nkv); bm must be 64; hd 64, or 128 (its own kernel: 32-key tiles, half blocks).
 */
int a8_prefill_attn(const void *q, int64_t s_qr, int64_t s_qh, int R,
                    const void *kc, const void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                    int cache_rows, int cache_len,
                    void *out, int64_t s_or, int64_t s_oh,
                    const int32_t *bq0, const int32_t *bn, const int32_t *bslot,
                    const int32_t *bpos0, int nblk, int bm,
                    int nq, int group, int hd, float scale, void *stream);

/*
 * a8_prefill_attn with q formed from the qkv rows inside the launch: no counterpart in the reference, which
 * writes q with bias_rope_store and reads it back in prefill_attention (serve/fast_engine.py:127-132 with
 * fast_kernels.py:179-187 and 350-358). Paired with a8_bias_rope_store(qo = NULL), the admission step neither
 * writes nor re-reads q. The query operands are exactly the q bias_rope_store would write: x = f32(qkv) +
 * f32(bias), rotate_half RoPE from the tables' row at the query position (block start bpos0 + row within the
 * block), rounded to bf16 with the store's arithmetic -- so the outputs are the bits of the two calls, for
 * finite qkv / bias and query positions inside [0, n_tab) (a query at a position outside the tables attends
 * with q = 0; the two-call path leaves its q unwritten).
 * qkv     [R, (nq + 2*nkv) * hd] row stride s_qkv (columns contiguous); bias [(nq + 2*nkv) * hd] or NULL
 * cos_tab, sin_tab [n_tab, hd] row stride s_cs (>= hd; n_tab * s_cs * 2 bytes below 2^32)
 * Other arguments: those of a8_prefill_attn. hd 64 only.
 */
int a8_prefill_attn_qkv(const void *qkv, int64_t s_qkv, const void *bias,
                        const void *cos_tab, const void *sin_tab, int64_t s_cs, int n_tab, int R,
                        const void *kc, const void *vc, int64_t s_kb, int64_t s_kh, int64_t s_ks,
                        int cache_rows, int cache_len,
                        void *out, int64_t s_or, int64_t s_oh,
                        const int32_t *bq0, const int32_t *bn, const int32_t *bslot,
                        const int32_t *bpos0, int nblk, int bm,
                        int nq, int group, int hd, float scale, void *stream);

/*
 * A voice prefix's K and V into the cache rows of the requests that use it, one launch for all layers
 * and slots. Replaces the two index-puts of serve/fast_engine.py:1102-1103 (FastEngine._prefill step 1:
 * kc_all[:, idx, :, :Lp] = k.unsqueeze(1), vc_all likewise), whose k / v come from _prefix_kv
 * (fast_engine.py:1073-1087).
 *
 * k, v            [layers, nkv, Lp, hd] strides (s_l, s_h, s_p, 1)
 * kc_all, vc_all  [layers, cache_rows, nkv, cache_len, hd] strides (d_l, d_r, d_h, d_p, 1) (shared)
 * slots           [n] int32: kc_all[l, slots[i], h, p] = k[l, h, p] and vc_all likewise, p < Lp.
 *                 A slot outside [0, cache_rows) is skipped (the reference would raise).
 * Positions must be contiguous rows on both sides (s_p == d_p == hd; hd a multiple of 8 up to 256);
 * Lp <= cache_len.
 */
int a8_prefix_copy(const void *k, const void *v, int64_t s_l, int64_t s_h, int64_t s_p,
                   void *kc_all, void *vc_all, int64_t d_l, int64_t d_r, int64_t d_h, int64_t d_p,
                   const int32_t *slots, int n, int layers, int nkv, int Lp, int hd, int cache_rows,
                   int cache_len, void *stream);

/*
 * The slow-AR layer's steps around the attention (the widening beside the path):
 * a8_rmsnorm replaces serve/fast_kernels.py:49-69 (rmsnorm, kernel 30-46): for each of `rows` rows of
 * width N (a multiple of 8, <= 2048), with residual != NULL: h = bf16(f32(x) + f32(residual)) is
 * written to res_out (may alias residual) and normalised; else h = x. y = bf16(f32(w) *
 * f32(bf16(f32(h) * rsqrt(mean(f32(h)^2) + eps)))). x, residual, y, res_out row strides sx, sr, sy, sro.
 * a8_silu_mul replaces serve/fast_kernels.py:537-545 (silu_mul, kernel 526-534): gu [rows, 2I] row
 * stride s_gu -> y [rows, I] row stride s_y, y = bf16(f32(bf16(g / (1 + exp(-g)))) * f32(u)) with
 * g = gu[:, :I], u = gu[:, I:]; I a multiple of 8.
 */
int a8_rmsnorm(const void *x, int64_t sx, const void *residual, int64_t sr, const void *w, void *y, int64_t sy,
               void *res_out, int64_t sro, int rows, int N, float eps, void *stream);
int a8_silu_mul(const void *gu, int64_t s_gu, void *y, int64_t s_y, int rows, int I, void *stream);

/*
 * Small-M GEMM for the slow-AR layer's projections (qkv, o, w13, w2 at the decode tick's token count):
 * out[M, N] = bf16(x[M, K] . w[N, K]^T), fp32 accumulation. Takes the small-M side of the reference's
 * per-shape GEMM choice (serve/fast_kernels.py:413-519, GemmDispatch.__call__: cuBLAS or a tuned Triton
 * linear_triton, 395-410), which the package's GemmDispatch makes between this and hipBLASLt by timing.
 * x [M, K] row stride ldx, w [N, K] row stride ldw (row-major: nn.Linear's weight), out [M, N] row stride ldo.
 * M <= 192, K a multiple of 64, N a multiple of 8, 16-byte aligned pointers, leading dims multiples of 8 and
 * at least the row length; else A8_EUNSUP / A8_EALIGN (the caller takes its library GEMM).
 * splits: k ranges computed by separate workgroups (1 = none; clamped to K / 64, then to the count that gives
 * every range a chunk: splits_used). With more than one, ws (16-byte aligned, >= 4096 + splits_used * M * N * 4
 * bytes, else A8_EWSPACE) holds 1024 32-bit tile counters in its first 4096 bytes, then the fp32 partials; the
 * last workgroup of each tile to finish sums them in a fixed order, in the same launch: deterministic. The
 * counters must be zero before a workspace's first use (allocate it zeroed); every call leaves them zero.
 * mblocks: row blocks the M token rows are split into (1 = all rows in each workgroup; a block holds an even
 * number of 16-row subtiles, so fewer blocks may be used), for more workgroups where N is narrow. Neither
 * changes the result. Two calls sharing ws must not overlap in time.
 */
int a8_gemm_small(const void *x, int64_t ldx, const void *w, int64_t ldw, void *out, int64_t ldo,
                  void *ws, int64_t ws_bytes, int M, int N, int K, int splits, int mblocks, void *stream);
/*
 * The w13 projection with the gated activation in its epilogue: out[M, I] = silu_mul(x . w13^T), w13 [2I, K]
 * = [gate; up] rows (row stride ldw), the product rounded to bf16 as a8_gemm_small's, then a8_silu_mul's
 * arithmetic (serve/fast_kernels.py:526-545): the same bits as a8_gemm_small followed by a8_silu_mul, in one
 * launch (the reference's SiLU-mul after its w13 GEMM, serve/fast_engine.py:135). M <= 192, K a multiple
 * of 64, I of 8; mblocks as for a8_gemm_small; no k splits.
 */
int a8_gemm_silu_small(const void *x, int64_t ldx, const void *w13, int64_t ldw, void *out, int64_t ldo, int M, int I,
                       int K, int mblocks, void *stream);
/*
 * The projections with the slow-AR layer's residual RMSNorm folded into them, so that the norm takes no launch of
 * its own (the reference runs rmsnorm, serve/fast_kernels.py:30-69, between its GEMMs, serve/fast_engine.py:131-137;
 * no counterpart entry point in the reference). Shapes, splits, ws and mblocks as a8_gemm_small; gated != 0: w =
 * [gate; up] (N = 2I rows), out [M, I] with a8_gemm_silu_small's epilogue (one split, N a multiple of 16).
 *   res_add != 0: out [M, N] is the residual stream, updated in place: out = bf16(f32(bf16(x . w^T)) + f32(out))
 *     -- the product rounded as a8_gemm_small's, then rmsnorm's residual add, the same bits. ss_out (optional,
 *     N a multiple of 32): fp32 [M][N / 32], the sums of squares of the new stream per 32-column group.
 *   ss_in (optional; not with res_add): x is a raw residual stream h and w carries the norm weight (w[n][k] =
 *     bf16(w[n][k] norm_w[k])); the fp32 products are scaled by rsqrt(sum_{j < ss_n} ss_in[m][j] / K + eps)
 *     before the rounding (ss_n a multiple of 4, <= 32; ss_in 16-byte aligned, row stride ss_n): the RMSNorm's
 *     1 / rms without the reference's two intermediate bf16 roundings, within their rounding noise.
 */
int a8_gemm_small_norm(const void *x, int64_t ldx, const void *w, int64_t ldw, void *out, int64_t ldo, void *ws,
                       int64_t ws_bytes, int M, int N, int K, int splits, int mblocks, int gated, int res_add,
                       float *ss_out, const float *ss_in, int ss_n, float eps, void *stream);
/*
 * a8_gemm_small_norm with `pf_slices` more grid slices of workgroups that only read [pf, pf + pf_bytes) once and
 * end (no counterpart in the reference): the next product's weights go into the memory-side cache while this
 * product runs; pf_sink a 16-byte device word the read may write in a case that practically never happens.
 */
int a8_gemm_small_norm_pf(const void *x, int64_t ldx, const void *w, int64_t ldw, void *out, int64_t ldo, void *ws,
                          int64_t ws_bytes, int M, int N, int K, int splits, int mblocks, int gated, int res_add,
                          float *ss_out, const float *ss_in, int ss_n, float eps, const void *pf, int64_t pf_bytes,
                          void *pf_sink, int pf_slices, void *stream);

/*
 * The streaming vocoder's channels-last convolutions (the codec decoder's default conv path,
 * serve/fast_engine.py:218-233), fp16 storage:
 * a8_conv_cl replaces serve/fast_kernels.py:600-623 (conv_cl, kernel 551-597): for rows (b, t), t < TR,
 *   y[b, t*ph + p, n] = bias[n] + sum_{j < taps} sum_k x[b, t + j*dil, k] w[p, j, k, n] (+ res[b, t*ph + p, n]),
 *   n < Cout; x [B, Tin, Cin] (Tin >= TR + (taps-1) dil, Cin a multiple of 8), w [ph, taps, Cin, cout_w]
 *   (cout_w >= Cout, a multiple of 8; last dim contiguous), bias [Cout] or NULL, res like y or NULL.
 *   snake_a / snake_ib (fp32 [Cin]) or NULL: x -> x + ib sin(a x)^2 (fp16) on the load (Cin <= 1024;
 *   wider inputs take snake_cat first). fp32 accumulation.
 *   ws / ws_bytes: an optional 16-byte aligned device workspace; with a8_conv_cl_ws_bytes(...) bytes the
 *   kernel may split K across workgroups (fixed-order fp32 sums: the same result with or without it).
 * a8_conv_cl_ws_bytes: the workspace a8_conv_cl would use for these sizes (0: none). No counterpart in the
 *   reference (its Triton conv splits nothing); lets the caller allocate from its own pool.
 * a8_snake_cat replaces serve/fast_kernels.py:718-729 (snake_cat, kernel 695-715):
 *   y[b] = concat(state[b] (CTX rows), snake(x[b]) (T rows)), C a multiple of 8; a / ib NULL: no snake.
 */
int a8_conv_cl(const void *x, int64_t s_xb, int64_t s_xt, const void *w, int64_t s_wp, int64_t s_wt, int64_t s_wc,
               int cout_w, const void *bias, const void *res, int64_t s_rb, int64_t s_rt, void *y, int64_t s_yb,
               int64_t s_yt, const float *snake_a, const float *snake_ib, int B, int Tin, int TR, int Cin, int Cout,
               int taps, int dil, int ph, void *ws, int64_t ws_bytes, void *stream);
int64_t a8_conv_cl_ws_bytes(int B, int TR, int Cin, int Cout, int taps, int ph);
int a8_snake_cat(const void *x, int64_t s_xb, int64_t s_xt, const void *state, int64_t s_sb, int64_t s_st,
                 const float *a, const float *ib, void *y, int64_t s_yb, int64_t s_yt, int B, int T, int CTX, int C,
                 void *stream);
/*
 * a8_snake_cat that also writes the next context (no counterpart entry point in the reference, which copies
 * it after the conv, serve/fast_engine.py:232): y as a8_snake_cat, and state[b] <- y[b, T .. T + CTX) in the same
 * launch (each old state row is read, then rewritten, by the same thread). Needs T >= CTX (else A8_EUNSUP).
 */
int a8_snake_cat_refresh(const void *x, int64_t s_xb, int64_t s_xt, void *state, int64_t s_sb, int64_t s_st,
                         const float *a, const float *ib, void *y, int64_t s_yb, int64_t s_yt, int B, int T, int CTX,
                         int C, void *stream);
/*
 * The codec decoder's last conv with what surrounds it, in one launch (no counterpart entry point in the
 * reference, which runs serve/fast_engine.py:228-233 -- snake_cat, conv_cl into one output channel, the state
 * copy -- and then y[..., 0].float().tanh() at 310): y[b, t] = tanh(f32(fp16(bias[0] + sum_{j < taps} sum_k
 * xin[b, t + j, k] w[j, k]))) with xin = [state[b] | snake(x[b])] (snake as a8_snake_cat's, fp32 sums), and
 * state[b] <- xin[b, T .. T + CTX). x [B, T, Cin] fp16 (row strides s_xb, s_xt); state [>=B, CTX, Cin] fp16,
 * activated, CTX = taps - 1 <= T; a / ib fp32 [Cin]; w [taps, Cin] fp16 contiguous; bias fp16 [1] or NULL;
 * y [B, T] fp32, row stride s_yb. Cin a multiple of 8 up to 128, taps up to 8; else A8_EUNSUP.
 */
int a8_conv_out_tanh(const void *x, int64_t s_xb, int64_t s_xt, void *state, int64_t s_sb, int64_t s_st,
                     const float *a, const float *ib, const void *w, const void *bias, float *y, int64_t s_yb,
                     int B, int T, int CTX, int Cin, int taps, void *stream);

/*
 * a8_ru_cl replaces serve/fast_kernels.py:679-692 (ru_fused, kernel 626-676; used by _FusedRU,
 * serve/fast_engine.py:235-273): one whole residual unit in one launch, for rows (b, t), t < TR:
 *   h = b1 + sum_{j < taps} xin[b, t + j*dil] w1[j]            (fp32, never stored)
 *   y[b, t, n] = res[b, t, n] + b2[n] + sum_k fp16(h + ib2 sin(a2 h)^2)[k] w2[k, n]
 * xin [B, Tin, C] the activated input ([state | snake1(x)]: a8_snake_cat's output, Tin >= TR + (taps-1) dil),
 * w1 [taps, C, C] (tap stride s_wt, row stride s_wc = C) and w2 [C, C] fp16 [k][n] rows, b1 / b2 fp16 [C]
 * (b1 8-byte aligned), a2 / ib2 fp32 [C] (16-byte aligned), res the unit's raw input. fp32 accumulation.
 * C must be 96, 192 or 384 (one workgroup holds a row's channels): else A8_EUNSUP.
 */
int a8_ru_cl(const void *xin, int64_t s_xb, int64_t s_xt, const void *w1, int64_t s_wt, int64_t s_wc, const void *b1,
             const float *a2, const float *ib2, const void *w2, const void *b2, const void *res, int64_t s_rb,
             int64_t s_rt, void *y, int64_t s_yb, int64_t s_yt, int B, int Tin, int TR, int C, int taps, int dil,
             void *stream);

#ifdef __cplusplus
}
#endif

#endif /* A8ATTN_H */
