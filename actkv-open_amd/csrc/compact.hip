// Conflict-free in-place compaction of a paged KV cache (ActKV Algorithm 4)
// for gfx950: plan, row moves and block reclaim in one launch.
//
// Reference: actkv/kernels/compaction.py:44-106 and actkv/paged.py:125-139.
// The reference plans on the host with torch.nonzero (two host syncs), then
// launches one Triton program per copy pair.  Here every workgroup of the
// single launch rebuilds the plan for its request from the packed keep bits:
// an LDS exclusive scan of per-word popcounts gives rank(pos) = #kept in
// [0, pos), from which
//   B = rank(Y*bs), start = (Y - ceil(B/bs)) * bs, end = start + B,
//   pair i: src = select1(i < K(start) ? i : i + K(end) - K(start))
//           dst = select0(i + start - K(start))
// (select1/select0 = binary search of the scan + in-word bit select).  The
// workgroup then moves its pairs' rows in its group of planes with 16-byte
// vector loads/stores.  src and dst never intersect, so no move reads a row
// that another move writes, within one plane or across planes.
#include "common.h"

#include <algorithm>

namespace actkv {

constexpr int CT = 256;        // threads per compaction workgroup
constexpr int MAX_PAIRS = 64;  // pairs per workgroup tile

struct CompactArgs {
  unsigned char *kv;
  int64_t planes, sp, ss, row_bytes, num_blocks;
  const uint32_t *bits;
  int64_t bits_sr;
  int R;
  const int32_t *seq_used;
  const int32_t *bt;
  int64_t bt_sr;
  int BS;
  int64_t *perm;
  int64_t perm_sr;
  const uint8_t *pin_in;
  int64_t pin_sr;
  const int32_t *pin_count;  // instead of pin_in: positions < pin_count[r] are pinned
  uint8_t *pin_out;
  int64_t pout_sr;
  int32_t *table_out;
  int64_t tout_sr;
  int32_t *freed;
  int64_t freed_sr;
  int64_t *src_out, *dst_out;
  int64_t pairs_sr;
  int32_t *counts;
  int do_copy, P, PG, max_words, max_kept;
};

// Exclusive scan of popcounts of words[0..nw) into pre[0..nw]; pre[nw] = total.
// Each thread sums a contiguous run of words; runs are scanned with DPP wave
// scans and one LDS pass over the CT/64 wave totals.
__device__ void scan_words(const uint32_t *words, uint32_t *pre, int nw) {
  __shared__ uint32_t wsum[CT / 64];
  const int per = (nw + CT - 1) / CT;
  const int lo = threadIdx.x * per, hi = min(lo + per, nw);
  uint32_t s = 0;
  for (int w = lo; w < hi; ++w) s += __popc(words[w]);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint32_t inc = wave_scan_u32(s, 0u, OpAdd());
  if (lane == 63) wsum[wv] = inc;
  __syncthreads();
  uint32_t run = inc - s;
  for (int i = 0; i < wv; ++i) run += wsum[i];
  for (int w = lo; w < hi; ++w) {
    pre[w] = run;
    run += __popc(words[w]);
  }
  if (threadIdx.x == CT - 1) pre[nw] = run;
  __syncthreads();
}

// #kept in [0, pos), 0 <= pos <= nw*32
__device__ __forceinline__ uint32_t rank1(const uint32_t *words, const uint32_t *pre, int nw,
                                          int pos) {
  const int w = pos >> 5, b = pos & 31;
  if (w >= nw) return pre[nw];
  return pre[w] + (b ? __popc(words[w] & ((1u << b) - 1u)) : 0u);
}

// position of the k-th (0-based) kept bit
__device__ __forceinline__ int select1(const uint32_t *words, const uint32_t *pre, int nw,
                                       uint32_t k) {
  int lo = 0, hi = nw - 1;  // largest w with pre[w] <= k
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (pre[mid] <= k) lo = mid; else hi = mid - 1;
  }
  return lo * 32 + select_bit(words[lo], (int)(k - pre[lo]));
}

// position of the k-th (0-based) non-kept bit
__device__ __forceinline__ int select0(const uint32_t *words, const uint32_t *pre, int nw,
                                       uint32_t k) {
  int lo = 0, hi = nw - 1;  // largest w with 32*w - pre[w] <= k
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((uint32_t)(mid * 32) - pre[mid] <= k) lo = mid; else hi = mid - 1;
  }
  return lo * 32 + select_bit(~words[lo], (int)(k - ((uint32_t)(lo * 32) - pre[lo])));
}

// Streaming copies: every moved row is read once and written once, so both
// sides use non-temporal accesses (no L2 allocation for the destination lines,
// which a write-allocate would otherwise fetch from HBM first).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <typename U>
__device__ __forceinline__ void copy_rows(unsigned char *kv, int64_t sp, int64_t ss,
                                          int64_t row_bytes, const int64_t *src_slot,
                                          const int64_t *dst_slot, int np, int64_t p0, int npl) {
  // items = npl planes x np pairs x units; < 2^31 by construction of the
  // tile shape (np <= 64, npl <= 65535 groups' worth, row <= 2^16 units).
  const int units = (int)(row_bytes / sizeof(U));
  const int per_plane = np * units;
  const int items = per_plane * npl;
  constexpr int UNR = 8;
  for (int base = threadIdx.x; base < items; base += CT * UNR) {
    U v[UNR];
    unsigned char *dptr[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int it = base + u * CT;
      dptr[u] = nullptr;
      if (it < items) {
        const int pl = it / per_plane;
        const int rem = it - pl * per_plane;
        const int pr = rem / units;
        const int unit = rem - pr * units;
        const int64_t s = src_slot[pr], d = dst_slot[pr];
        if (s >= 0 && d >= 0) {
          const int64_t poff = (p0 + pl) * sp + (int64_t)unit * sizeof(U);
          v[u] = __builtin_nontemporal_load((const U *)(kv + poff + s * ss));
          dptr[u] = kv + poff + d * ss;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u)
      if (dptr[u]) __builtin_nontemporal_store(v[u], (U *)dptr[u]);
  }
}

// Pinned flag of old logical position pos of request r (pcount: pin_count[r]).
__device__ __forceinline__ uint8_t pin_of(const CompactArgs &a, int r, int pos, int pcount) {
  return a.pin_in ? a.pin_in[(int64_t)r * a.pin_sr + pos] : (uint8_t)(pos < pcount);
}

// grid (tiles, plane groups, R), CT threads, dynamic LDS 2*max_words words.  The
// length and the pin count are read together at the start.
template <typename U>
__global__ void __launch_bounds__(CT) compact_kernel(CompactArgs a) {
  extern __shared__ uint32_t sm[];
  __shared__ int64_t src_slot[MAX_PAIRS], dst_slot[MAX_PAIRS];
  const int r = blockIdx.z;
  const int pcount = a.pin_count ? a.pin_count[r] : 0;
  const int S = max(a.seq_used[r], 0);
  const int Y = (S + a.BS - 1) / a.BS;
  const int nw = (Y * a.BS + 31) >> 5;
  if (nw > a.max_words) {  // longer than the launch's max_seq: left untouched, reported as -2
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0 && a.counts) {
      int32_t *c = a.counts + (int64_t)r * 4;
      c[0] = -2; c[1] = -2; c[2] = -2; c[3] = -2;
    }
    return;
  }
  uint32_t *words = sm;
  uint32_t *pre = sm + a.max_words;
  const uint32_t *brow = a.bits + (int64_t)r * a.bits_sr;
  const int32_t *btr = a.bt + (int64_t)r * a.bt_sr;
  for (int w = threadIdx.x; w < nw; w += CT) words[w] = brow[w];
  __syncthreads();
  scan_words(words, pre, nw);
  const int B = (int)pre[nw];
  const int X = (B + a.BS - 1) / a.BS;
  const int drop = Y - X;
  const int start = drop * a.BS, end = start + B;
  if (B > a.max_kept) {  // grid too small for this request: left untouched, reported as -1
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0 && a.counts) {
      int32_t *c = a.counts + (int64_t)r * 4;
      c[0] = -1; c[1] = -1; c[2] = -1; c[3] = -1;
    }
    return;
  }
  const uint32_t Kst = rank1(words, pre, nw, start), Ken = rank1(words, pre, nw, end);
  const int M = (int)(Kst + ((uint32_t)B - Ken));
  const int i0 = blockIdx.x * a.P;
  const bool lead = blockIdx.y == 0;

  if (threadIdx.x < a.P) {
    const int i = i0 + threadIdx.x;
    int64_t sslot = -1, dslot = -1;
    if (i < M) {
      const uint32_t k1 = (uint32_t)i < Kst ? (uint32_t)i : (uint32_t)i + (Ken - Kst);
      const int src = select1(words, pre, nw, k1);
      const int dst = select0(words, pre, nw, (uint32_t)i + ((uint32_t)start - Kst));
      const int64_t sb = btr[src / a.BS], db = btr[dst / a.BS];
      if (sb >= 0 && sb < a.num_blocks && db >= 0 && db < a.num_blocks) {
        sslot = sb * a.BS + src % a.BS;
        dslot = db * a.BS + dst % a.BS;
      }
      if (lead) {
        if (a.perm) a.perm[(int64_t)r * a.perm_sr + (dst - start)] = src;
        if (a.pin_out) a.pin_out[(int64_t)r * a.pout_sr + (dst - start)] = pin_of(a, r, src, pcount);
        if (a.src_out) a.src_out[(int64_t)r * a.pairs_sr + i] = sslot;
        if (a.dst_out) a.dst_out[(int64_t)r * a.pairs_sr + i] = dslot;
      }
    }
    src_slot[threadIdx.x] = sslot;
    dst_slot[threadIdx.x] = dslot;
    // kept positions inside the window stay where they are
    const int j = i0 + threadIdx.x;
    if (lead && j < B) {
      const int pos = start + j;
      if ((words[pos >> 5] >> (pos & 31)) & 1u) {
        if (a.perm) a.perm[(int64_t)r * a.perm_sr + j] = pos;
        if (a.pin_out) a.pin_out[(int64_t)r * a.pout_sr + j] = pin_of(a, r, pos, pcount);
      }
    }
  }
  if (lead && blockIdx.x == 0) {
    for (int x = threadIdx.x; x < X; x += CT)
      if (a.table_out) a.table_out[(int64_t)r * a.tout_sr + x] = btr[drop + x];
    for (int j = threadIdx.x; j < drop; j += CT)
      if (a.freed) a.freed[(int64_t)r * a.freed_sr + j] = btr[drop - 1 - j];
    if (threadIdx.x == 0 && a.counts) {
      int32_t *c = a.counts + (int64_t)r * 4;
      c[0] = B; c[1] = M; c[2] = drop; c[3] = X;
    }
  }
  __syncthreads();
  if (!a.do_copy || i0 >= M) return;
  const int np = min(a.P, M - i0);
  const int64_t p0 = (int64_t)blockIdx.y * a.PG;
  const int npl = (int)std::min<int64_t>(a.PG, a.planes - p0);
  if (npl <= 0) return;
  copy_rows<U>(a.kv, a.sp, a.ss, a.row_bytes, src_slot, dst_slot, np, p0, npl);
}

// grid (ceil(n_pairs/P), plane groups), CT threads.
template <typename U>
__global__ void __launch_bounds__(CT) copy_slots_kernel(unsigned char *kv, int64_t planes,
                                                        int64_t sp, int64_t ss, int64_t row_bytes,
                                                        int64_t num_slots, const int64_t *src,
                                                        const int64_t *dst, int64_t n_pairs,
                                                        int P, int PG) {
  __shared__ int64_t src_slot[MAX_PAIRS], dst_slot[MAX_PAIRS];
  const int64_t i0 = (int64_t)blockIdx.x * P;
  if (threadIdx.x < P) {
    const int64_t i = i0 + threadIdx.x;
    int64_t s = -1, d = -1;
    if (i < n_pairs) {
      s = src[i];
      d = dst[i];
      if (s < 0 || s >= num_slots || d < 0 || d >= num_slots) s = d = -1;
    }
    src_slot[threadIdx.x] = s;
    dst_slot[threadIdx.x] = d;
  }
  __syncthreads();
  const int np = (int)std::min<int64_t>(P, n_pairs - i0);
  const int64_t p0 = (int64_t)blockIdx.y * PG;
  const int npl = (int)std::min<int64_t>(PG, planes - p0);
  if (np <= 0 || npl <= 0) return;
  copy_rows<U>(kv, sp, ss, row_bytes, src_slot, dst_slot, np, p0, npl);
}

// grid (ceil(W/256), L, R): per-token metadata follows the compaction
// permutation: dst[l, r, i] = src[l, r, perm[r, i]] for i < kept[r], 0 for
// kept[r] <= i < W (a permutation entry outside [0, W) also reads as 0).
__global__ void __launch_bounds__(256) gather_tokens_kernel(const float *src, int64_t s_sl, int64_t s_sr,
                                                            float *dst, int64_t d_sl, int64_t d_sr, int W,
                                                            const int64_t *perm, int64_t perm_sr,
                                                            const int32_t *kept) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int l = blockIdx.y, r = blockIdx.z;
  if (i >= W) return;
  float v = 0.f;
  if (i < kept[r]) {
    const int64_t j = perm[(int64_t)r * perm_sr + i];
    if (j >= 0 && j < W) v = src[(int64_t)l * s_sl + (int64_t)r * s_sr + j];
  }
  dst[(int64_t)l * d_sl + (int64_t)r * d_sr + i] = v;
}

// Widest access unit dividing every byte offset the copy touches.
static int unit_bytes(const void *base, int64_t sp, int64_t ss, int64_t row_bytes) {
  const uint64_t m = (uint64_t)(uintptr_t)base | (uint64_t)sp | (uint64_t)ss | (uint64_t)row_bytes;
  if ((m & 15u) == 0) return 16;
  if ((m & 7u) == 0) return 8;
  if ((m & 3u) == 0) return 4;
  if ((m & 1u) == 0) return 2;
  return 1;
}

// Pairs per tile and planes per group: about 16k workgroups, each moving 32 KiB
// .. 2 MiB.  Many small workgroups keep the tail of the launch short (every CU
// stays busy until the end); the per-workgroup plan (scan + selects) stays a
// small fraction of its row moves.
static void copy_shape(int64_t max_pairs, int64_t planes, int64_t row_bytes, int *P, int *PG) {
  const int64_t bytes = std::max<int64_t>(1, max_pairs) * planes * row_bytes;
  int64_t per_wg = std::max<int64_t>(32 * 1024, std::min<int64_t>(2048 * 1024, bytes / 16384));
  int64_t pairs_cap = std::max<int64_t>(1, per_wg / std::max<int64_t>(1, row_bytes));
  int p = (int)std::min<int64_t>(MAX_PAIRS, std::max<int64_t>(4, std::min<int64_t>(pairs_cap, max_pairs)));
  int64_t pg = std::max<int64_t>(1, per_wg / ((int64_t)p * row_bytes));
  *P = p;
  *PG = (int)std::min<int64_t>(planes, pg);
}

}  // namespace actkv

using namespace actkv;

extern "C" int actkv_gather_tokens(const float *src, int64_t src_sl, int64_t src_sr, float *dst,
                                   int64_t dst_sl, int64_t dst_sr, int L, int R, int W,
                                   const int64_t *perm, int64_t perm_sr, const int32_t *kept,
                                   void *stream) {
  if (!src || !dst || !perm || !kept || L < 1 || R < 1 || W < 0) return ACTKV_ERR_INVALID_ARG;
  if (src == dst) return ACTKV_ERR_INVALID_ARG;  // a gather cannot run in place
  if (L > 65535 || R > 65535) return ACTKV_ERR_UNSUPPORTED;
  if (W == 0) return ACTKV_OK;
  dim3 grid((unsigned)((W + 255) / 256), (unsigned)L, (unsigned)R);
  hipLaunchKernelGGL(gather_tokens_kernel, grid, dim3(256), 0, (hipStream_t)stream, src, src_sl, src_sr, dst,
                     dst_sl, dst_sr, W, perm, perm_sr, kept);
  return actkv_check_launch();
}

extern "C" int actkv_copy_slots(void *kv_flat, int64_t planes, int64_t stride_plane_bytes,
                                int64_t stride_slot_bytes, int64_t row_bytes, int64_t num_slots,
                                const int64_t *src, const int64_t *dst, int64_t n_pairs,
                                void *stream) {
  if (n_pairs == 0) return ACTKV_OK;
  if (!kv_flat || !src || !dst || n_pairs < 0 || planes < 1 || row_bytes < 1 || num_slots < 1)
    return ACTKV_ERR_INVALID_ARG;
  int P, PG;
  copy_shape(n_pairs, planes, row_bytes, &P, &PG);
  const int64_t gx = (n_pairs + P - 1) / P, gy = (planes + PG - 1) / PG;
  if (gx > 0x7fffffffLL || gy > 65535) return ACTKV_ERR_UNSUPPORTED;
  dim3 grid((unsigned)gx, (unsigned)gy);
  hipStream_t st = (hipStream_t)stream;
  unsigned char *kv = (unsigned char *)kv_flat;
  switch (unit_bytes(kv_flat, stride_plane_bytes, stride_slot_bytes, row_bytes)) {
#define ACTKV_COPY(UT)                                                                        \
  hipLaunchKernelGGL(copy_slots_kernel<UT>, grid, dim3(CT), 0, st, kv, planes,                \
                     stride_plane_bytes, stride_slot_bytes, row_bytes, num_slots, src, dst, \
                     n_pairs, P, PG);                                                       \
  break
    case 16: ACTKV_COPY(u32x4);
    case 8: ACTKV_COPY(u32x2);
    case 4: ACTKV_COPY(uint32_t);
    case 2: ACTKV_COPY(uint16_t);
    default: ACTKV_COPY(uint8_t);
#undef ACTKV_COPY
  }
  return actkv_check_launch();
}

extern "C" int actkv_compact(void *kv, int64_t planes, int64_t stride_plane_bytes,
                             int64_t stride_slot_bytes, int64_t row_bytes, int64_t num_blocks,
                             const uint32_t *keep_bits, int64_t bits_sr, int R,
                             const int32_t *seq_used, const int32_t *block_table, int64_t bt_sr,
                             int block_size, int64_t *perm_out, int64_t perm_sr,
                             const uint8_t *pinned_in, int64_t pin_sr, const int32_t *pin_count,
                             uint8_t *pinned_out,
                             int64_t pout_sr, int32_t *table_out, int64_t tout_sr,
                             int32_t *freed_out, int64_t freed_sr, int64_t *src_out,
                             int64_t *dst_out, int64_t pairs_sr, int32_t *counts_out, int do_copy,
                             int max_seq, int max_kept, void *stream) {
  if (!keep_bits || !seq_used || !block_table || R < 1 || block_size < 1 || max_seq < 0 ||
      max_kept < 0)
    return ACTKV_ERR_INVALID_ARG;
  if (do_copy && (!kv || planes < 1 || row_bytes < 1)) return ACTKV_ERR_INVALID_ARG;
  // pinned_out needs exactly one source: a mask or a leading count
  if (pinned_in && pin_count) return ACTKV_ERR_INVALID_ARG;
  if ((pinned_out != nullptr) != (pinned_in != nullptr || pin_count != nullptr)) return ACTKV_ERR_INVALID_ARG;
  const int64_t padded = ((int64_t)(max_seq + block_size - 1) / block_size) * block_size;
  const int64_t max_words = (padded + 31) / 32;
  const size_t shm = (size_t)(2 * max_words + 2) * sizeof(uint32_t);
  if (shm > 64 * 1024) return ACTKV_ERR_UNSUPPORTED;
  CompactArgs a;
  a.kv = (unsigned char *)kv; a.planes = planes; a.sp = stride_plane_bytes;
  a.ss = stride_slot_bytes; a.row_bytes = row_bytes; a.num_blocks = num_blocks;
  a.bits = keep_bits; a.bits_sr = bits_sr; a.R = R; a.seq_used = seq_used;
  a.bt = block_table; a.bt_sr = bt_sr; a.BS = block_size;
  a.perm = perm_out; a.perm_sr = perm_sr; a.pin_in = pinned_in; a.pin_sr = pin_sr; a.pin_count = pin_count;
  a.pin_out = pinned_out; a.pout_sr = pout_sr; a.table_out = table_out; a.tout_sr = tout_sr;
  a.freed = freed_out; a.freed_sr = freed_sr; a.src_out = src_out; a.dst_out = dst_out;
  a.pairs_sr = pairs_sr; a.counts = counts_out; a.do_copy = do_copy;
  a.max_words = (int)max_words + 1;
  a.max_kept = max_kept;
  int P, PG;
  copy_shape(max_kept, do_copy ? planes : 1, do_copy ? row_bytes : 2048, &P, &PG);
  if (!do_copy) { P = MAX_PAIRS; PG = 1; }
  a.P = P;
  a.PG = PG;
  const int64_t gx = std::max<int64_t>(1, ((int64_t)max_kept + P - 1) / P);
  const int64_t gy = do_copy ? (planes + PG - 1) / PG : 1;
  if (gx > 0x7fffffffLL || gy > 65535 || R > 65535) return ACTKV_ERR_UNSUPPORTED;
  dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)R);
  hipStream_t st = (hipStream_t)stream;
  switch (do_copy ? unit_bytes(kv, stride_plane_bytes, stride_slot_bytes, row_bytes) : 16) {
#define ACTKV_COMPACT(UT) \
  hipLaunchKernelGGL(compact_kernel<UT>, grid, dim3(CT), shm, st, a); break
    case 16: ACTKV_COMPACT(u32x4);
    case 8: ACTKV_COMPACT(u32x2);
    case 4: ACTKV_COMPACT(uint32_t);
    case 2: ACTKV_COMPACT(uint16_t);
    default: ACTKV_COMPACT(uint8_t);
#undef ACTKV_COMPACT
  }
  return actkv_check_launch();
}

extern "C" const char *actkv_error_string(int status) {
  switch (status) {
    case ACTKV_OK: return "ACTKV_OK";
    case ACTKV_ERR_INVALID_ARG: return "ACTKV_ERR_INVALID_ARG";
    case ACTKV_ERR_UNSUPPORTED: return "ACTKV_ERR_UNSUPPORTED";
    case ACTKV_ERR_WORKSPACE: return "ACTKV_ERR_WORKSPACE";
    case ACTKV_ERR_LAUNCH: return "ACTKV_ERR_LAUNCH";
  }
  return "ACTKV_ERR_UNKNOWN";
}

extern "C" const char *actkv_version(void) { return "actkv-hip 0.1 gfx950"; }
