/*
 * actkv.h -- C ABI of the MI355X (gfx950) ActKV eviction hot path.
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * launches asynchronously on the caller's HIP stream, allocates no memory and
 * returns an int status (ACTKV_OK or an ACTKV_ERR_* code).  Caller-owned
 * workspaces are sized with actkv_workspace_size().  No entry point
 * synchronises the device.
 *
 * Layout vocabulary (the reference's paged cache, actkv/paged.py:3, :54-55):
 *   kv          [layers, 2, num_blocks, block_size, n_kv_heads, head_dim]
 *   block_table [R, max_blocks] int32   logical block -> physical block
 *   seq_used    [R] int32               valid tokens per request
 *   scores/out  [layers, R, n_kv_heads, W] float32, W >= max_blocks*block_size
 *
 * Citations are path:line in the reference repository (Maurya30/actkv-open).
 */
#ifndef ACTKV_H_
#define ACTKV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */
#define ACTKV_OK 0
#define ACTKV_ERR_INVALID_ARG 1   /* a size, stride, pointer or dtype is invalid   */
#define ACTKV_ERR_UNSUPPORTED 2   /* valid, but outside what the kernels handle    */
#define ACTKV_ERR_WORKSPACE 3     /* workspace missing or smaller than required    */
#define ACTKV_ERR_LAUNCH 4        /* hipLaunchKernel / hipGetLastError failed      */

/* element types */
#define ACTKV_F32 0
#define ACTKV_F16 1
#define ACTKV_BF16 2

/* head_reduce (actkv/paged.py:32-36) */
#define ACTKV_REDUCE_MEAN 0
#define ACTKV_REDUCE_MAX 1

/* workspace kinds for actkv_workspace_size */
#define ACTKV_WS_KEEP_MASK 0

/* Human-readable name of a status code (static storage). */
const char *actkv_error_string(int status);

/* Library version string, e.g. "actkv-hip 0.1 gfx950". */
const char *actkv_version(void);

/*
 * actkv_action_scores -- LSE-recovery scoring (ActKV Algorithm 3).
 *
 * Replaces actkv/kernels/lse_attn.py:133-163 (`action_scores`) and its
 * Triton kernel lse_attn.py:85-130.  The reference folds ONE action query per
 * request per call; this entry point folds N queries (and L layers) in one
 * launch.  For every layer l, request r, KV head h and token t < seq_used[r]:
 *
 *   p_n[t] = max_{g<G} exp(scale * q[l,r,n,h*G+g,:] . k[l,t,h,:] - lse[l,r,n,h*G+g])
 *   out[l,r,h,t] <- running mean of p_0..p_{nq-1} continuing from n_seen[r]
 *                   (== the reference's nq successive folds, lse_attn.py:127-130)
 *
 * then n_seen[r] += nq (lse_attn.py:162).  nq = n_valid ? n_valid[r] : N.
 * Query n of request r only sees tokens t < kv_len[r*N + n] when kv_len is
 * non-NULL (causal action region); unseen tokens contribute 0 to the mean.
 * Slots t >= seq_used[r] are not touched (lse_attn.py:111, :130).
 *
 * q     : dtype q_dtype, [L, R, N, Hq, D], strides q_sl q_sr q_sn q_sh, unit last
 * kv    : dtype kv_dtype, K plane of layer l at kv + l*kv_sl; V plane ignored;
 *         block stride kv_sb, slot stride kv_ss, head stride kv_sh, unit last.
 *         num_blocks bounds every physical id read from block_table.
 * lse   : float32 [L, R, N, Hq], strides lse_sl lse_sr lse_sn, unit last
 * out   : float32 [L, R, Hkv, W], strides out_sl out_sr out_sh, unit last,
 *         W >= max_blocks*block_size (checked)
 * scale : softmax scale (the reference default is head_dim^-0.5, lse_attn.py:148)
 * bf16/fp16 q and K of one dtype with D = 128 or 64 and Hq/Hkv from 1 to 16 run on the
 * matrix cores (groups of 3, 5-7 and 9-15 laid out as 4, 8 and 16 rows per query, the extra rows
 * padding; 512/G' queries per launch for the laid-out group G', more as several
 * launches); every other case uses float32 dot products.
 */
int actkv_action_scores(
    const void *q, int q_dtype, int64_t q_sl, int64_t q_sr, int64_t q_sn, int64_t q_sh,
    const void *kv, int kv_dtype, int64_t kv_sl, int64_t kv_sb, int64_t kv_ss, int64_t kv_sh,
    int64_t num_blocks,
    const int32_t *block_table, int64_t bt_sr, int max_blocks,
    const int32_t *seq_used,
    const float *lse, int64_t lse_sl, int64_t lse_sr, int64_t lse_sn,
    float *out, int64_t out_sl, int64_t out_sr, int64_t out_sh, int64_t out_width,
    int32_t *n_seen, const int32_t *n_valid, const int32_t *kv_len,
    int L, int R, int N, int Hq, int Hkv, int D, int block_size,
    float scale, void *stream);

/*
 * actkv_copy_slots -- row copies kv_flat[p, dst[i], :] = kv_flat[p, src[i], :]
 * for every plane p < planes and pair i < n_pairs.
 *
 * Replaces actkv/kernels/compaction.py:96-106 (`apply_copies`) and its Triton
 * kernel compaction.py:79-93.  src and dst are int64 slot indices; the caller
 * guarantees src and dst are disjoint (compaction.py:13, :72-74), which makes
 * every copy order-independent.  Strides are in BYTES (64-bit), row_bytes is
 * the contiguous row length.  Slots must lie in [0, num_slots).
 */
int actkv_copy_slots(void *kv_flat, int64_t planes, int64_t stride_plane_bytes,
                     int64_t stride_slot_bytes, int64_t row_bytes, int64_t num_slots,
                     const int64_t *src, const int64_t *dst, int64_t n_pairs,
                     void *stream);

/*
 * actkv_keep_mask -- scores -> keep mask (protected tokens + top-`budget` others).
 *
 * Replaces actkv/paged.py:23-46 (`keep_mask_from_scores`), batched over R
 * requests.  scores is [L, R, H, W] of dtype scores_dtype with element strides
 * s_sl s_sr s_sh and unit last stride; the reference's 1-D case is L=H=1 and
 * the 2-D [Hkv, S] case is L=1.  Per request r with S = seq_used[r]:
 *
 *   s[t] = mean_l( reduce_h scores[l,r,h,t] )      reduce = mean | max
 *
 * with the float32 summation order of torch's CPU `mean` (a cascade of
 * 16-row blocks over its vectorized columns: whole 32-column blocks, or the
 * first 4 columns of a 4-7-column row; its 4-way interleaved order for the
 * others) and a correctly rounded division, so s is bit-identical to the
 * reference on the same scores.  keep = protected  OR  the k = clamp(budget[r], 0, #unprotected)
 * largest s among unprotected tokens; among equal scores at the boundary the
 * lower index wins.  protected is a per-request count of leading tokens
 * (protected_count) or a bool mask (protected_mask, row stride pm_sr); exactly
 * one of the two may be non-NULL (both NULL: nothing protected).
 *
 * keep (bool bytes, row stride keep_sr) receives S entries per request.
 * keep_bits (row stride bits_sr in uint32 words) receives the same mask packed
 * LSB-first, zero-padded to a whole number of blocks of block_size tokens: the
 * input of actkv_compact.  Either may be NULL, not both.
 * workspace must hold actkv_workspace_size(ACTKV_WS_KEEP_MASK, R, max_seq)
 * bytes (the per-token keys); it needs no initialisation.  Calls that share a
 * workspace must be stream-ordered.  Limits: L <= 256 (ACTKV_ERR_UNSUPPORTED
 * beyond).
 */
int actkv_keep_mask(const void *scores, int scores_dtype, int64_t s_sl, int64_t s_sr,
                    int64_t s_sh, int L, int H, int R, const int32_t *seq_used,
                    const int32_t *budget, const int32_t *protected_count,
                    const uint8_t *protected_mask, int64_t pm_sr, int head_reduce,
                    uint8_t *keep, int64_t keep_sr, uint32_t *keep_bits, int64_t bits_sr,
                    int block_size, int max_seq, void *workspace, size_t workspace_bytes,
                    void *stream);

/*
 * actkv_keep_mask_noalloc -- actkv_keep_mask without a caller workspace.
 *
 * No counterpart in the reference: an addition for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid allocation).  Same
 * arguments, results and errors as actkv_keep_mask, minus the workspace: the per-token
 * keys and the per-64-token candidate statistics live in a file-scope device array of
 * ACTKV_KEEP_MASK_SCRATCH_BYTES bytes per GPU, held from the library's load until the
 * process ends.  Calls whose actkv_workspace_size(ACTKV_WS_KEEP_MASK, R, max_seq) exceeds
 * it return ACTKV_ERR_WORKSPACE and launch nothing.  The array's address is looked up on
 * the current device at its first call there, so `stream` must belong to the current
 * device.  Every call on a GPU shares that GPU's array (each call writes every part it
 * reads first, so a call never sees the last one's contents): calls that may overlap on one
 * GPU race and must be ordered on one stream.
 */
#define ACTKV_KEEP_MASK_SCRATCH_BYTES ((size_t)8 << 20)
int actkv_keep_mask_noalloc(const void *scores, int scores_dtype, int64_t s_sl, int64_t s_sr,
                            int64_t s_sh, int L, int H, int R, const int32_t *seq_used,
                            const int32_t *budget, const int32_t *protected_count,
                            const uint8_t *protected_mask, int64_t pm_sr, int head_reduce,
                            uint8_t *keep, int64_t keep_sr, uint32_t *keep_bits, int64_t bits_sr,
                            int block_size, int max_seq, void *stream);

/*
 * actkv_pack_keep -- keep mask bytes [R, >=S] (a nonzero byte is a kept token, as a
 * bool mask's 1) -> packed bits (LSB-first), zero beyond seq_used[r] up to a whole
 * number of blocks, plus the popcount of each request's mask in kept_out[r]
 * (optional).  Support for actkv_compact when the caller holds a bool mask
 * (actkv/paged.py:125-132).
 */
int actkv_pack_keep(const uint8_t *keep, int64_t keep_sr, int R, const int32_t *seq_used,
                    int block_size, uint32_t *keep_bits, int64_t bits_sr,
                    int32_t *kept_out, int max_seq, void *stream);

/*
 * actkv_compact -- fused conflict-free in-place compaction (ActKV Algorithm 4)
 * of R requests in ONE launch: plan + row moves + block reclaim.
 *
 * Replaces actkv/paged.py:125-139 (`PagedKVCache.compact`) together with
 * actkv/kernels/compaction.py:44-69 (`plan_compaction`) and :96-106
 * (`apply_copies`).  Per request r with S = seq_used[r], B = popcount of its
 * keep bits, Y = ceil(S/bs), X = ceil(B/bs), start = (Y-X)*bs, end = start+B:
 *   dst = non-kept logical positions in [start, end), ascending
 *   src = kept logical positions outside [start, end), ascending
 *   the i-th src row moves onto the i-th dst row in every one of the `planes`
 *   planes of kv (all layers' K and V), physical slot = table[l/bs]*bs + l%bs.
 * src and dst are disjoint, so no copy reads a row another copy writes; rows
 * in reclaimed blocks are read within this launch and only handed out by
 * allocations that are stream-ordered after it.
 * Outputs (each optional, NULL to skip; row strides in elements):
 *   perm_out   int64 [R, >=B]: new logical -> old logical (compaction.py:67-68)
 *   pinned_in/pinned_out bool: pinned_out[r, j] = pinned_in[r, perm[j]] (paged.py:156);
 *              with pin_count instead of pinned_in (int32 [R], a request's first
 *              pin_count[r] tokens pinned, paged.py:150-151):
 *              pinned_out[r, j] = perm[j] < pin_count[r].  At most one of the two.
 *   table_out  int32 [R, >=X]: block_table[r, drop:drop+X] (paged.py:136)
 *   freed_out  int32 [R, >=drop]: freed blocks in free-list push order,
 *              i.e. block_table[r, drop-1-j] (paged.py:135-137)
 *   src_out/dst_out int64 [R, >=M]: physical slots of the plan (compaction.py:69)
 *   counts_out int32 [R, 4]: {B, M, drop, X}; a request the launch does not move is
 *              reported as {-1, -1, -1, -1} (B > max_kept) or {-2, -2, -2, -2}
 *              (seq_used[r] > max_seq), and its rows, perm and tables are not written
 * do_copy = 0 computes the plan outputs without moving rows (plan_compaction).
 * kv strides are in BYTES; row_bytes is the contiguous row (n_kv_heads*head_dim*esize).
 * max_kept bounds B over all requests (sizes the grid; checked in-kernel).
 */
int actkv_compact(void *kv, int64_t planes, int64_t stride_plane_bytes,
                  int64_t stride_slot_bytes, int64_t row_bytes, int64_t num_blocks,
                  const uint32_t *keep_bits, int64_t bits_sr, int R, const int32_t *seq_used,
                  const int32_t *block_table, int64_t bt_sr, int block_size,
                  int64_t *perm_out, int64_t perm_sr, const uint8_t *pinned_in, int64_t pin_sr,
                  const int32_t *pin_count, uint8_t *pinned_out, int64_t pout_sr,
                  int32_t *table_out, int64_t tout_sr,
                  int32_t *freed_out, int64_t freed_sr, int64_t *src_out, int64_t *dst_out,
                  int64_t pairs_sr, int32_t *counts_out, int do_copy, int max_seq, int max_kept,
                  void *stream);

/* Bytes of caller workspace an entry point needs (kind = ACTKV_WS_*). */
size_t actkv_workspace_size(int kind, int R, int max_seq);

/*
 * actkv_gather_tokens -- per-token metadata follows a compaction: for every
 * layer l < L and request r < R,
 *   dst[l, r, i] = src[l, r, perm[r, i]]  for i < kept[r]
 *   dst[l, r, i] = 0                      for kept[r] <= i < W
 * (perm as written by actkv_compact: new logical -> old logical; an entry
 * outside [0, W) reads as 0).  The reference permutes such state by indexing
 * with the permutation (actkv/kernels/compaction.py:16-18,
 * actkv/eviction.py:222-224).  src and dst are float32 with strides (sl, sr)
 * and a unit last stride, and must not overlap.
 */
int actkv_gather_tokens(const float *src, int64_t src_sl, int64_t src_sr, float *dst,
                        int64_t dst_sl, int64_t dst_sr, int L, int R, int W, const int64_t *perm,
                        int64_t perm_sr, const int32_t *kept, void *stream);

/*
 * actkv_lrfu_update -- LRFU keep-score update (ActKV Algorithm 1 steps 2-4)
 * of the paged cache, one (layer, request) segment per workgroup.
 *
 * Replaces actkv/eviction.py:209-218 (ActionLRFU.update_scores) with its
 * nucleus actkv/eviction.py:36-50 (top_p_mask), for a paged cache whose
 * per-token action scores come from actkv_action_scores.  For layer l,
 * request r, S = seq_used[r], P = protected_count[r] (0 if NULL), or, with
 * protected_mask (bool [R, >=S], row stride pm_sr) instead, the pinned tokens
 * (excluded from the nucleus, ks untouched; at most one of the two):
 *   act[t] = mean (torch CPU float32 order) or max over the H heads of
 *            scores[l, r, h, t]                               (eviction.py:20-33)
 *   hit    = over t in [P, S): the entries taken in descending act order
 *            (equal values: lower index first) until the running sum reaches
 *            top_p * total (float64 running sums compared as float32, as
 *            torch's cumsum), positive entries only; no hits when
 *            active[r] == 0 or total <= 0                   (eviction.py:36-50)
 *   ks[l, r, t] = decay * ks[l, r, t]  (+ act[t] where hit), t in [P, S)
 * ks entries below P and at or past S are not touched.
 * scores float32 [L, R, H, >=S] (strides s_sl s_sr s_sh, unit last);
 * ks float32 [L, R, >=S] (strides ks_sl ks_sr, unit last), in place;
 * hit_out (optional) bool [L, R, >=S]: the hit mask over [P, S).
 * workspace: actkv_lrfu_workspace_size(L, R, max_seq) bytes, any contents.
 */
int actkv_lrfu_update(const float *scores, int64_t s_sl, int64_t s_sr, int64_t s_sh, int L, int H,
                      int R, const int32_t *seq_used, const int32_t *protected_count,
                      const uint8_t *protected_mask, int64_t pm_sr,
                      const int32_t *active, float *ks, int64_t ks_sl, int64_t ks_sr,
                      uint8_t *hit_out, int64_t hit_sl, int64_t hit_sr, float decay, float top_p,
                      int head_reduce, int max_seq, void *workspace, size_t workspace_bytes,
                      void *stream);

/* Workspace bytes for actkv_lrfu_update (one float per layer, request and token). */
size_t actkv_lrfu_workspace_size(int L, int R, int max_seq);

/*
 * actkv_paged_attention -- paged attention with the log-sum-exp by-product (the
 * lse producer that actkv_action_scores consumes).
 *
 * Replaces actkv/kernels/lse_attn.py:42-60 (`paged_decode_attention_ref`, the
 * stand-in for a paged FlashAttention backend) and actkv/paged.py:115-118
 * (`decode_attention`).  The reference takes one query per request; this entry
 * point takes N queries per request and L layers.  For layer l, request r,
 * query n < nq (nq = n_valid ? n_valid[r] : N), query head hq (KV head hq / G):
 *
 *   s_t = scale * q[l,r,n,hq,:] . k[l,t,hq/G,:]   for t < lim
 *   lse[l,r,n,hq]   = logsumexp_t s_t
 *   out[l,r,n,hq,:] = sum_t softmax(s)_t v[l,t,hq/G,:]
 *
 * lim = seq_used[r], or min(kv_len[r*N + n], seq_used[r]) when kv_len is
 * non-NULL (causal limits).  A query with lim = 0 gets lse = -inf, out = 0.
 * Rows n >= nq are not written.
 *
 * q   : dtype q_dtype, [L, R, N, Hq, D], strides q_sl q_sr q_sn q_sh, unit last
 * kv  : dtype kv_dtype; K plane of layer l at kv + l*kv_sl, V plane at
 *       kv + l*kv_sl + kv_sv; block stride kv_sb, slot stride kv_ss, head
 *       stride kv_sh, unit last.  num_blocks bounds every physical id read from
 *       block_table (ids outside the pool are skipped).
 * out : float32 [L, R, N, Hq, D], strides o_sl o_sr o_sn o_sh, unit last
 * lse : float32 [L, R, N, Hq], strides lse_sl lse_sr lse_sn, unit last
 * bf16/fp16 with D = 128 or 64 (any Hq/Hkv) run on the matrix cores
 * (each probability enters the P.V product as a hi and a lo term in the cache
 * dtype, P = hi + lo to about 2^-16 relative, float32 accumulation); every other
 * case uses float32 dot products.  D <= 512.
 * workspace: optional, actkv_paged_attention_workspace_size(...) bytes, any
 * contents.  With it, long sequences are split into token chunks attended in
 * parallel and merged by a second launch (flash-decoding); without it (NULL or
 * smaller), every sequence is attended by one workgroup per row group.
 */
int actkv_paged_attention(
    const void *q, int q_dtype, int64_t q_sl, int64_t q_sr, int64_t q_sn, int64_t q_sh,
    const void *kv, int kv_dtype, int64_t kv_sl, int64_t kv_sv, int64_t kv_sb, int64_t kv_ss,
    int64_t kv_sh, int64_t num_blocks,
    const int32_t *block_table, int64_t bt_sr, int max_blocks,
    const int32_t *seq_used, const int32_t *n_valid, const int32_t *kv_len,
    float *out, int64_t o_sl, int64_t o_sr, int64_t o_sn, int64_t o_sh,
    float *lse, int64_t lse_sl, int64_t lse_sr, int64_t lse_sn,
    int L, int R, int N, int Hq, int Hkv, int D, int block_size,
    float scale, void *workspace, size_t workspace_bytes, void *stream);

/* Workspace bytes that let actkv_paged_attention split long sequences (0: it
 * does not split this shape). */
size_t actkv_paged_attention_workspace_size(int L, int R, int N, int Hq, int Hkv, int D,
                                            int max_blocks, int block_size);

/*
 * actkv_append -- write appended tokens into the paged cache, every layer and both
 * planes, for R requests in one launch.
 *
 * Replaces the data movement of actkv/paged.py:76-84 (`PagedKVCache.append`):
 *   kv[l, 0, slot(starts[r] + i)] = k[l, src_off[r] + i].to(kv dtype), same for V,
 *   slot(t) = block_table[r, t / block_size] * block_size + t % block_size,
 * for i < counts[r]; total = sum of counts.  The blocks must already be in the
 * table: allocation (paged.py:67-74, the free-block stack) is the caller's, as in
 * the reference.  Conversions round to nearest even (torch's .to()).
 * kv : dtype kv_dtype; K plane of layer l at kv + l*kv_sl, V plane + kv_sv; block,
 *      slot and head strides kv_sb kv_ss kv_sh, unit last (elements).
 * k, v : dtype src_dtype, [L, >=total, Hkv, D]; strides (k_sl, k_sn, k_sh) and
 *      (v_sl, v_sn, v_sh), unit last.
 * starts, counts : int32 [R]; src_off : int64 [R]; block_table int32 [R, bt_sr].
 * bad (optional): set to 1 if a destination block is missing from the table or
 *      outside the pool (that token is skipped).
 * Rows that are 16-byte aligned with D a multiple of 8 move 8 elements per thread;
 * any other layout one element per thread.  Strides may be 0 (broadcast sources).
 */
int actkv_append(void *kv, int kv_dtype, int64_t kv_sl, int64_t kv_sv, int64_t kv_sb,
                 int64_t kv_ss, int64_t kv_sh, int64_t num_blocks,
                 const void *k, const void *v, int src_dtype,
                 int64_t k_sl, int64_t k_sn, int64_t k_sh, int64_t v_sl, int64_t v_sn, int64_t v_sh,
                 int L, int Hkv, int D, int R, const int32_t *starts, const int32_t *counts,
                 const int64_t *src_off, int64_t total,
                 const int32_t *block_table, int64_t bt_sr, int max_blocks, int block_size,
                 int32_t *bad, void *stream);

/*
 * actkv_slot_map -- out[i] = table_row[t / block_size] * block_size + t % block_size
 * for t = start + i, i < n (int64; -1 past the table's nblocks entries).
 * Replaces actkv/paged.py:93-97 (`slot_map`, which is the start = 0 case).
 */
int actkv_slot_map(const int32_t *table_row, int nblocks, int start, int n, int block_size,
                   int64_t *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* ACTKV_H_ */
