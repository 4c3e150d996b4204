// Scores -> keep mask (protected tokens + top-`budget` others) for gfx950.
//
// Reference: actkv/paged.py:23-46 (keep_mask_from_scores).  Two launches,
// batched over requests:
//   keys   : grid (ceil(max_seq/TOK), R), 512 threads, TOK = 128 tokens per
//            block up to 120 layers, 64 up to 256.  Per token, reduce KV
//            heads (mean|max) then average layers, with the float32 order of
//            torch's CPU `mean` so s[t] is bit-identical to the reference, and
//            write an order-preserving uint32 key (0 marks a protected token).
//   select : one 1024-thread block per request, its keys in LDS (chunks of
//            32768 tokens beyond that).  Finds the exact k-th
//            largest key by narrowing a window of key values (2048 bins per
//            pass over the candidates' own range; past one chunk, the window's
//            candidates in LDS once they fit), and the index cut among tied keys (lower index
//            wins), then writes
//            keep[t] = protected | key > thr | (key == thr & t < cut),
//            packed LSB-first into 32-bit words for actkv_compact too.
// The keys pass reads the scores once from HBM with every CU busy; the selection
// works on data one CU holds, and the launch boundary between the two is what
// makes every block's keys visible to the request's selecting block.
//
// torch CPU sum order (aten SumKernel cascade_sum, pinned by the oracle tests):
// for a reduction over n rows of a column block, the column's value is a
// cascade of 16-row blocks (level_power 4) when the column lies in the
// vectorized body (torch_body_end), and the "row_sum" 4-way interleaved order
// for the other columns.  Division by the row count is IEEE (div_, not a
// reciprocal multiply).
#include "common.h"
#include "torch_order.h"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace actkv {

constexpr int HIST_BINS = 2048;
constexpr int KT = 512;                 // threads per keys block
constexpr int TOK_WIDE = 128;           // tokens per keys block up to MAX_LAYERS_WIDE layers
constexpr int TOK_NARROW = 64;          // ... and up to MAX_LAYERS (one wave of tokens)
constexpr int SEL_T = 1024;             // threads per select block
constexpr int CAND_CAP = 1536;          // window candidates the select block holds in LDS
constexpr int MAX_LAYERS_WIDE = 120;    // [L][TOK] layer values fit 64 KiB of LDS:
constexpr int MAX_LAYERS = 256;         // 120 x 128 and 256 x 64 floats

struct KeepArgs {
  const void *scores;
  int64_t s_sl, s_sr, s_sh;
  int L, H, R;
  const int32_t *seq_used, *budget, *prot_count;
  const uint8_t *prot_mask;
  int64_t pm_sr;
  int head_reduce;
  uint8_t *keep;      // optional when bits is given
  int64_t keep_sr;
  uint32_t *bits;     // optional
  int64_t bits_sr;
  int BS, max_seq;
  uint32_t *keys;     // [R, keys_sr], keys_sr = max_seq rounded up to a multiple of 4
  int64_t keys_sr;
  uint4 *stats;       // [R, stats_sr]: per 64 tokens {candidates, min key, max key, 0}
  int64_t stats_sr;   // ceil(max_seq / 64)
};

__device__ __forceinline__ bool is_protected(const KeepArgs &a, int r, int t) {
  if (a.prot_mask) return a.prot_mask[(int64_t)r * a.pm_sr + t] != 0;
  if (a.prot_count) return t < a.prot_count[r];
  return false;
}

// Block-wide helpers (any multiple of 64 threads up to 1024).
__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t *scratch) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[w] = v;
  __syncthreads();
  uint32_t tot = 0;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) tot += scratch[i];
  __syncthreads();
  return tot;
}

// The select kernel keeps a request's keys in LDS, KCHUNK at a time (the whole
// request up to 32768 tokens), so every pass over them is a short loop of LDS
// reads; longer requests are walked chunk by chunk from memory.
constexpr int KCHUNK = 32768;

__device__ __forceinline__ void load_chunk(uint32_t *skeys, const uint32_t *keys, int c0, int n) {
  const int n4 = n >> 2;
  const uint4 *src = (const uint4 *)(keys + c0);   // c0 % 4 == 0, rows 16-byte aligned
  constexpr int U = 8;                             // 16-byte loads in flight per thread: 32768
                                                   // keys in one round with 1024 threads (in-bounds
                                                   // clamped reads past n4 are not stored)
  for (int i = threadIdx.x; i < n4; i += U * blockDim.x) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = src[min(i + u * (int)blockDim.x, n4 - 1)];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i + u * (int)blockDim.x < n4) ((uint4 *)skeys)[i + u * blockDim.x] = v[u];
  }
  for (int i = 4 * n4 + threadIdx.x; i < n; i += blockDim.x) skeys[i] = keys[c0 + i];
}

// Bit i of the low byte of x moved to bit 4i.
__device__ __forceinline__ uint32_t spread4(uint32_t x) {
  x &= 0xFFu;
  x = (x | (x << 12)) & 0x000F000Fu;
  x = (x | (x << 6)) & 0x03030303u;
  x = (x | (x << 3)) & 0x11111111u;
  return x;
}

// Visit (key, t) of n keys of a chunk held in LDS: 16-byte reads, two per
// thread in flight.
template <typename F>
__device__ __forceinline__ void visit_chunk(const uint32_t *skeys, int c0, int n, F f) {
  const int n4 = n >> 2;
  const uint4 *k4 = (const uint4 *)skeys;
  for (int i = threadIdx.x; i < n4; i += 2 * blockDim.x) {
    const int j = i + blockDim.x;
    const uint4 v0 = k4[i];
    const uint4 v1 = j < n4 ? k4[j] : make_uint4(0, 0, 0, 0);
    f(v0.x, c0 + 4 * i); f(v0.y, c0 + 4 * i + 1); f(v0.z, c0 + 4 * i + 2); f(v0.w, c0 + 4 * i + 3);
    if (j < n4) { f(v1.x, c0 + 4 * j); f(v1.y, c0 + 4 * j + 1); f(v1.z, c0 + 4 * j + 2); f(v1.w, c0 + 4 * j + 3); }
  }
  for (int t = 4 * n4 + threadIdx.x; t < n; t += blockDim.x) f(skeys[t], c0 + t);
}

// Visit (key, t) for every t < S.  When the request is longer than one chunk,
// every call reloads the chunks (the caller has synchronised after its last use).
template <typename F>
__device__ __forceinline__ void visit_keys(uint32_t *skeys, const uint32_t *keys, int S, F f) {
  if (S <= KCHUNK) {
    visit_chunk(skeys, 0, S, f);
    return;
  }
  for (int c0 = 0; c0 < S; c0 += KCHUNK) {
    const int n = min(KCHUNK, S - c0);
    __syncthreads();
    load_chunk(skeys, keys, c0, n);
    __syncthreads();
    visit_chunk(skeys, c0, n, f);
  }
}

// Count the keys of an LDS-resident request (S <= KCHUNK) that fall in the
// window [base, base + 2^wbits), wbits <= 21, into hist[(key - base) >> sh].
// For a narrow window: each thread tests its keys 32 at a time and issues LDS
// atomics only for the few inside, so a wave makes a handful of atomic
// instructions instead of one per key slot (each costs LDS pipe time however
// few lanes it carries).  Called by every thread of the block.
__device__ __forceinline__ void count_window_sparse(const uint32_t *skeys, int S, uint32_t base, int wbits,
                                                    int sh, uint32_t *hist) {
  const int n4 = S >> 2;
  const uint4 *k4 = (const uint4 *)skeys;
  const uint32_t width = 1u << wbits;
  auto in = [&](uint32_t key) -> uint32_t { return (uint32_t)((key != 0u) & (key - base < width)); };
  constexpr int U = 8;
  for (int i0 = 0; i0 < n4; i0 += U * blockDim.x) {
    uint32_t m = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * blockDim.x + threadIdx.x;
      const uint4 v = i < n4 ? k4[i] : make_uint4(0u, 0u, 0u, 0u);
      m |= (in(v.x) | (in(v.y) << 1) | (in(v.z) << 2) | (in(v.w) << 3)) << (4 * u);
    }
    while (m) {
      const int j = __builtin_ctz(m);
      m &= m - 1;
      const uint32_t key = skeys[4 * (i0 + (j >> 2) * blockDim.x + threadIdx.x) + (j & 3)];
      atomicAdd(&hist[(key - base) >> sh], 1u);
    }
  }
  for (int t = 4 * n4 + threadIdx.x; t < S; t += blockDim.x) {
    const uint32_t key = skeys[t];
    if (in(key)) atomicAdd(&hist[(key - base) >> sh], 1u);
  }
}

// Bit width of x (0 for x == 0).
__device__ __forceinline__ int bit_width(uint32_t x) { return x ? 32 - __clz(x) : 0; }

// The bin holding the k-th largest element of hist[nbins] (LDS), 1 <= k <= total,
// in two barriers; *need = k - (elements in the bins above it).  Thread i of the
// NT-thread block owns nbins/NT bins from the top; DPP wave scans and the per-wave
// totals (wtot, 16-byte aligned, NT/64 entries) give each thread its exclusive
// count, and the one thread whose bins cross k resolves the bin.  Between the
// barriers it clears clear[0, nclear) (the next pass's counts).
template <int NT>
__device__ int find_bin(const uint32_t *hist, int nbins, uint32_t k, uint32_t *need, uint32_t *wtot,
                        uint32_t *found, uint32_t *clear, int nclear) {
  static_assert(NT % 256 == 0 && NT <= 1024, "wave totals are read four at a time");
  const int per = nbins / NT;
  const int top = nbins - 1 - (int)threadIdx.x * per;
  uint32_t c = 0;
  for (int j = 0; j < per; ++j) c += hist[top - j];
  const uint32_t inc = wave_scan_u32(c, 0u, OpAdd());
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 63) wtot[w] = inc;
  for (int i = threadIdx.x; i < nclear; i += NT) clear[i] = 0;
  __syncthreads();
  uint32_t before = 0;
#pragma unroll
  for (int q = 0; q < NT / 64; q += 4) {
    const uint4 x = *(const uint4 *)(wtot + q);
    before += (q < w ? x.x : 0u) + (q + 1 < w ? x.y : 0u) + (q + 2 < w ? x.z : 0u) + (q + 3 < w ? x.w : 0u);
  }
  const uint32_t excl = before + inc - c;   // elements in the bins above my range
  if (excl < k && excl + c >= k) {
    uint32_t above = excl;
    int b = top;
    for (int j = 0; j < per; ++j, --b) {
      if (above + hist[b] >= k) break;
      above += hist[b];
    }
    found[0] = (uint32_t)b;
    found[1] = k - above;
  }
  __syncthreads();
  *need = found[1];
  return (int)found[0];
}

// grid R, SEL_T threads: the selection and the write of request r's keep mask.
//
// The k-th largest candidate key (key != 0) is found by narrowing a window of
// key values: it starts as [min, max] of the candidates (from the keys kernel's
// per-64-token figures), and each pass splits the window into 2048 bins, counts
// the candidates per bin and keeps the bin holding the k-th largest.  Binning
// the keys' own range instead of fixed key bits spreads them over the bins even
// when the scores are concentrated (an average over many layers, heads and
// queries), which keeps the LDS atomics of the counting pass apart.  Once the
// window's candidates fit in LDS they are gathered there and the remaining
// passes touch only them.
//
// A request of up to KCHUNK tokens is resident: thread i holds the keys of
// tokens j*SEL_T + i (j < KPT) in registers, loaded while the statistics are
// reduced, and a token-ordered copy in LDS for the walks that go by index (the
// gather's read-back, ties, a window too wide to gather, the mask).  The first
// pass and the gather test the register keys; the mask is written with one
// ballot per 64 consecutive tokens, i.e. two whole words per wave.  The
// selection is bound by the VALU work per key on one CU, so each key is tested
// with as few operations as the case allows.  A longer request walks its keys
// from memory in LDS chunks.  The passes are arranged for few block barriers:
// the next pass's counts are cleared inside the bin search, counters are set
// before the first barrier.
constexpr int KPT = KCHUNK / SEL_T;     // keys per thread of a resident request

__global__ void __launch_bounds__(SEL_T) keep_select_kernel(KeepArgs a) {
  __shared__ __attribute__((aligned(16))) uint32_t skeys[KCHUNK];
  __shared__ uint32_t hist_a[HIST_BINS], hist_b[HIST_BINS];
  __shared__ uint2 cand[CAND_CAP];
  __shared__ uint32_t red[3][SEL_T / 64], found[2];
  __shared__ __attribute__((aligned(16))) uint32_t wtot[SEL_T / 64];
  __shared__ int ncand_s, ntie_s, cut_s;
  const int r = blockIdx.x;
  const int S = min(max(a.seq_used[r], 0), a.max_seq);
  if (S == 0) return;
  const uint32_t *keys = a.keys + (int64_t)r * a.keys_sr;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const bool resident = S <= KCHUNK;       // uniform over the block
  for (int b = threadIdx.x; b < HIST_BINS; b += blockDim.x) hist_a[b] = 0;
  if (threadIdx.x == 0) { ncand_s = 0; ntie_s = 0; cut_s = 0x7fffffff; }
  // candidates (unprotected tokens): count, smallest and largest key, from the
  // keys kernel's per-64-token figures, reduced in one barrier; their loads go
  // first, the keys' loads (clamped in bounds, zero past S) behind them
  const uint4 *st = a.stats + (int64_t)r * a.stats_sr;
  const int ngroups = (S + 63) / 64;
  const uint4 s0 = st[min((int)threadIdx.x, ngroups - 1)];
  uint32_t kr[KPT];
  if (resident) {
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int t = j * SEL_T + threadIdx.x;
      const uint32_t v = keys[min(t, S - 1)];
      kr[j] = t < S ? v : 0u;
    }
  }
  uint32_t cnt = 0, kmin = 0xFFFFFFFFu, kmax = 0;
  if ((int)threadIdx.x < ngroups) { cnt = s0.x; kmin = s0.y; kmax = s0.z; }
  for (int g = threadIdx.x + blockDim.x; g < ngroups; g += blockDim.x) {
    const uint4 v = st[g];
    cnt += v.x;
    kmin = min(kmin, v.y);
    kmax = max(kmax, v.z);
  }
  cnt = wave_scan_u32(cnt, 0u, OpAdd());
  kmin = wave_scan_u32(kmin, 0xFFFFFFFFu, OpMin());
  kmax = wave_scan_u32(kmax, 0u, OpMax());
  if (lane == 63) { red[0][wv] = cnt; red[1][wv] = kmin; red[2][wv] = kmax; }
  __syncthreads();
  if (resident) {
#pragma unroll
    for (int j = 0; j < KPT; ++j) skeys[j * SEL_T + threadIdx.x] = kr[j];   // read after later barriers
  }
  uint32_t cand_n = 0, lo = 0xFFFFFFFFu, hi = 0;
  for (int i = 0; i < SEL_T / 64; ++i) {
    cand_n += red[0][i];
    lo = min(lo, red[1][i]);
    hi = max(hi, red[2][i]);
  }
  const int bud = a.budget[r];
  const uint32_t k = bud <= 0 ? 0u : ((uint32_t)bud < cand_n ? (uint32_t)bud : cand_n);
  uint32_t thr = 0;
  int cut = 0;
  if (k == 0) {
    thr = 0xFFFFFFFFu;                       // no candidate kept (NaN keys == thr, t >= cut)
  } else if (k < cand_n) {
    // window [base, base + 2^wbits): the candidates ranked (need)-th from its top
    uint32_t base = lo, need = k, in_win = cand_n;
    int wbits = bit_width(hi - lo);          // hi - lo < 2^wbits
    bool in_lds = false;
    int nc = 0;
    uint32_t *cur = hist_a, *nxt = hist_b;   // cur is zero
    bool first = true;
    while (true) {
      const int sh = max(0, wbits - 11);     // 2048 bins of 2^sh keys
      auto count = [&](uint32_t key, int) {
        const uint32_t d = key - base;
        if (key != 0 && (wbits >= 32 || d < (1u << wbits))) atomicAdd(&cur[d >> sh], 1u);
      };
      if (in_lds) {
        for (int i = threadIdx.x; i < nc; i += blockDim.x) count(cand[i].x, (int)cand[i].y);
      } else if (resident && first) {
        // every candidate lies in [lo, hi]: only the protected tokens (key 0) are skipped
#pragma unroll
        for (int j = 0; j < KPT; ++j)
          if (kr[j] != 0u) atomicAdd(&cur[(kr[j] - base) >> sh], 1u);
      } else if (resident) {                 // a window too wide to gather (wbits <= 21)
        count_window_sparse(skeys, S, base, wbits, sh, cur);
      } else {
        visit_keys(skeys, keys, S, count);
      }
      __syncthreads();
      uint32_t need2;
      const int b = find_bin<SEL_T>(cur, HIST_BINS, need, &need2, wtot, found, nxt, HIST_BINS);
      in_win = cur[b];
      need = need2;
      base += (uint32_t)b << sh;
      wbits = sh;
      first = false;
      if (sh == 0) break;                    // the bin is one key value: the threshold
      if (!in_lds && in_win <= (uint32_t)CAND_CAP) {
        // gather the window's candidates (key, index) into LDS
        if (resident) {
          // key - base < lim: in the window and not 0 (base >= lo >= 1); a thread's
          // hits go to consecutive slots placed by a DPP scan, one shared-count
          // update per wave, the keys read back from the LDS copy
          const uint32_t lim = min(1u << wbits, 0u - base);
          uint32_t m = 0;
#pragma unroll
          for (int j = 0; j < KPT; ++j) m |= (uint32_t)(kr[j] - base < lim) << j;
          const uint32_t c = __popc(m);
          const uint32_t inc = wave_scan_u32(c, 0u, OpAdd());
          const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
          if (tot != 0) {                    // uniform over the wave
            uint32_t wb = 0;
            if (lane == 0) wb = (uint32_t)atomicAdd(&ncand_s, (int)tot);
            uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int)wb, 0) + inc - c;
            while (m) {
              const int j = __builtin_ctz(m);
              m &= m - 1;
              const int t = j * SEL_T + threadIdx.x;
              cand[o++] = make_uint2(skeys[t], (uint32_t)t);
            }
          }
        } else {
          visit_keys(skeys, keys, S, [&](uint32_t key, int t) {
            if (key != 0 && key - base < (1u << wbits)) cand[atomicAdd(&ncand_s, 1)] = make_uint2(key, (uint32_t)t);
          });
        }
        __syncthreads();
        nc = ncand_s;
        in_lds = true;
      }
      uint32_t *tmp = cur; cur = nxt; nxt = tmp;
    }
    thr = base;
    const uint32_t ties = in_win;            // candidates whose key == thr
    cut = 0x7fffffff;
    if (need < ties && (in_lds || resident) && ties <= (uint32_t)HIST_BINS) {
      // keep the `need` lowest-index tokens whose key == thr: the tied candidates'
      // indices are gathered from LDS and each finds its rank among them
      uint32_t *tie_t = nxt;
      if (in_lds) {
        for (int i = threadIdx.x; i < nc; i += blockDim.x)
          if (cand[i].x == thr) tie_t[atomicAdd(&ntie_s, 1)] = cand[i].y;
      } else {
        visit_chunk(skeys, 0, S, [&](uint32_t key, int t) {
          if (key == thr) tie_t[atomicAdd(&ntie_s, 1)] = (uint32_t)t;
        });
      }
      __syncthreads();
      const int nt = ntie_s;
      for (int i = threadIdx.x; i < nt; i += blockDim.x) {
        const uint32_t ti = tie_t[i];
        uint32_t rank = 0;
        for (int j = 0; j < nt; ++j) rank += tie_t[j] < ti;
        if (rank + 1 == need) cut_s = (int)ti + 1;
      }
      __syncthreads();
      cut = cut_s;
    } else if (need < ties) {
      // many ties: ordered block scan over the keys
      uint32_t running = 0;
      for (int base_t = 0; base_t < S; base_t += blockDim.x) {
        const int t = base_t + threadIdx.x;
        const bool f = t < S && keys[t] == thr;
        const unsigned long long bal = __ballot(f);
        __syncthreads();
        if (lane == 0) wtot[wv] = (uint32_t)__popcll(bal);
        __syncthreads();
        uint32_t before = running;
        for (int i = 0; i < wv; ++i) before += wtot[i];
        before += (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
        if (f && before + 1 == need) cut_s = t + 1;
        uint32_t tot = 0;
        for (int i = 0; i < SEL_T / 64; ++i) tot += wtot[i];
        running += tot;
        __syncthreads();
        if (running >= need) break;
      }
      __syncthreads();
      cut = cut_s;
    }
  }
  // (k == cand_n: thr = 0, cut = 0 keeps every token)
  // write: lane i of a wave tests token t0 + i of 64 consecutive tokens t0 (a
  // multiple of 64); the wave's ballot is words t0/32 and t0/32 + 1, stored by
  // lanes 0 and 1.  Without a tie cut and with thr >= 1 the test is one
  // subtraction and one compare: key - 1 >= thr - 1 keeps key 0 (protected,
  // wraps to the top) and every key >= thr.
  const int padded = ((S + a.BS - 1) / a.BS) * a.BS;
  const int nw = (padded + 31) >> 5;
  uint8_t *krow = a.keep ? a.keep + (int64_t)r * a.keep_sr : nullptr;
  uint32_t *brow = a.bits ? a.bits + (int64_t)r * a.bits_sr : nullptr;
  auto write_mask = [&](auto simple) {
    constexpr bool SIMPLE = decltype(simple)::value;
    // t = this lane's token; whole = every token of the wave's 64 is < S (uniform)
    auto one = [&](int t, uint32_t key, bool whole) {
      bool kp = SIMPLE ? (key - 1u >= thr - 1u) : ((key == 0u) | (key > thr) | ((key == thr) & (t < cut)));
      if (!whole) kp = kp & (t < S);
      const unsigned long long bal = __ballot(kp);
      if (krow && t < S) krow[t] = kp ? 1 : 0;
      if (brow && lane < 2) {
        const int w = ((t - lane) >> 5) + lane;
        if (w < nw) brow[w] = lane ? (uint32_t)(bal >> 32) : (uint32_t)bal;
      }
    };
    // the keys come from the LDS copy (a resident request's is whole), one chunk
    // of KCHUNK tokens at a time
    for (int c0 = 0; c0 < padded; c0 += KCHUNK) {
      const int n = min(KCHUNK, S - c0);     // keys of the chunk (n <= 0: padding only)
      if (!resident) {
        __syncthreads();
        if (n > 0) load_chunk(skeys, keys, c0, n);
        __syncthreads();
      }
      for (int j = 0; j < KPT; ++j) {
        const int tl = j * SEL_T + threadIdx.x;
        one(c0 + tl, tl < n ? skeys[tl] : 0u, c0 + (j + 1) * SEL_T <= S);
      }
    }
  };
  if (resident && cut == 0x7fffffff && thr != 0u) {
    // the common case, from the register keys: a wave's 64 tokens t0 + lane of
    // slot j give words t0/32 (lane 0) and t0/32 + 1 (lane 1)
    // the compare's lane mask is the ballot (no per-lane boolean); the lanes
    // past S are masked off with a mask built from the wave's first token
    const uint32_t thr1 = thr - 1u;
    const int wu = __builtin_amdgcn_readfirstlane(wv);
    const int bsh = 32 * (lane & 1);
    static_assert(2 * KPT == 64, "one word per lane");
    uint32_t myword = 0;
    auto slots = [&](auto wb) {
      constexpr bool WB = decltype(wb)::value;
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const int rem = S - (j * SEL_T + 64 * wu);     // tokens of the wave's 64 that are < S
        const unsigned long long valid = rem >= 64 ? ~0ull : rem <= 0 ? 0ull : (1ull << rem) - 1ull;
        const unsigned long long bal = __builtin_amdgcn_uicmp(kr[j] - 1u, thr1, 35 /* unsigned >= */) & valid;
        if (WB) {
          const int t = j * SEL_T + threadIdx.x;
          if (t < S) krow[t] = (uint8_t)((bal >> lane) & 1ull);
        }
        // lanes 2j and 2j + 1 keep slot j's two words: one store per wave at the end
        // (a store instruction costs the memory pipeline about as much for two
        // lanes as for 64)
        const uint32_t word = (uint32_t)(bal >> bsh);    // even lanes: low half, odd lanes: high half
        myword = (lane >> 1) == j ? word : myword;
      }
    };
    if (brow) {
      if (krow) slots(std::integral_constant<bool, true>());
      else slots(std::integral_constant<bool, false>());
      const int w = (lane >> 1) * (SEL_T / 32) + 2 * wv + (lane & 1);
      if (w < nw) brow[w] = myword;
      for (int w = KCHUNK / 32 + threadIdx.x; w < nw; w += blockDim.x) brow[w] = 0u;   // past the resident
    } else {                                                                            // span (a block size
      write_mask(std::integral_constant<bool, true>());                                 // not dividing it)
    }
  } else if (cut == 0x7fffffff && thr != 0u) {
    write_mask(std::integral_constant<bool, true>());
  } else {
    write_mask(std::integral_constant<bool, false>());
  }
}

// The end of every keys block: layer means of its tokens -> keys, and per 64
// tokens (one wave) the candidate count and the smallest and largest candidate
// key, which the select kernel reduces instead of passing over the keys.  lvals
// [L][TOK] holds the head-reduced score of each (layer, token) of the block.
template <int TOK>
__device__ __forceinline__ void write_keys(const KeepArgs &a, int r, int S, int t0, const float *lvals) {
  const int tok = threadIdx.x;
  if (tok >= TOK) return;                  // the first TOK / 64 waves, whole
  const int t = t0 + tok;
  uint32_t key = 0;
  if (t < S) {
    if (!is_protected(a, r, t)) {
      auto ld = [&](int l) { return lvals[l * TOK + tok]; };
      key = float_key(__fdiv_rn(torch_sum(ld, a.L, t < torch_body_end(S)), (float)a.L));
    }
    a.keys[(int64_t)r * a.keys_sr + t] = key;
  }
  const bool c = key != 0;                 // candidate keys are never 0
  const uint32_t mn = wave_min_u32(c ? key : 0xFFFFFFFFu), mx = wave_max_u32(key);
  const uint32_t n = (uint32_t)__popcll(__ballot(c));
  if ((tok & 63) == 0 && t < S) a.stats[(int64_t)r * a.stats_sr + t / 64] = make_uint4(n, mn, mx, 0u);
}

// float32 scores with 16-byte aligned token rows: thread (layer group tid/(TOK/4),
// quad tid%(TOK/4)) reduces the HH heads of 4 consecutive tokens with 16-byte loads,
// up to three layers' loads in flight at once.  Same per-token float order as the
// generic kernel (a 4-token quad lies wholly in or out of the torch body:
// torch_body_end is a multiple of 4).
template <int HH, int TOK>
__global__ void __launch_bounds__(KT) keep_vec4_kernel(KeepArgs a) {
  constexpr int QUADS = TOK / 4, LGROUPS = KT / QUADS;
  extern __shared__ __attribute__((aligned(16))) float lvals[];  // [L][TOK]
  const int r = blockIdx.y;
  const int S = min(max(a.seq_used[r], 0), a.max_seq);
  const int t0 = blockIdx.x * TOK;
  if (t0 >= S) return;
  const int quad = threadIdx.x % QUADS, lg = threadIdx.x / QUADS;
  const int tq = t0 + 4 * quad;
  const bool body4 = tq < torch_body_end(S);
  const float *sbase = (const float *)a.scores + (int64_t)r * a.s_sr + tq;
  const int nin = min(S - tq, 4);
  auto load4 = [&](const float *p) {
    if (nin >= 4) return *(const f32x4 *)p;
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < nin; ++j) x[j] = p[j];
    return x;
  };
  // layers whose loads are in flight together (16 heads: one, within the registers)
  constexpr int LIF = HH <= 8 ? 3 : 1;
  if (tq < S) {
    for (int l0 = lg; l0 < a.L; l0 += LGROUPS * LIF) {
      f32x4 hv[LIF][HH];
#pragma unroll
      for (int it = 0; it < LIF; ++it) {
        const int l = l0 + LGROUPS * it;
        if (l < a.L) {
#pragma unroll
          for (int hh = 0; hh < HH; ++hh) hv[it][hh] = load4(sbase + (int64_t)l * a.s_sl + (int64_t)hh * a.s_sh);
        }
      }
#pragma unroll
      for (int it = 0; it < LIF; ++it) {
        const int l = l0 + LGROUPS * it;
        if (l >= a.L) continue;
        f32x4 v;
        if (a.head_reduce == ACTKV_REDUCE_MAX) {
          v = hv[it][0];
#pragma unroll
          for (int hh = 1; hh < HH; ++hh) {
            v[0] = nanmax(v[0], hv[it][hh][0]); v[1] = nanmax(v[1], hv[it][hh][1]);
            v[2] = nanmax(v[2], hv[it][hh][2]); v[3] = nanmax(v[3], hv[it][hh][3]);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            auto ld = [&](int hh) { return hv[it][hh][j]; };
            v[j] = __fdiv_rn(torch_sum(ld, HH, body4), (float)HH);
          }
        }
        *(f32x4 *)&lvals[l * TOK + 4 * quad] = v;
      }
    }
  }
  __syncthreads();
  write_keys<TOK>(a, r, S, t0, lvals);
}

// Any score dtype, head count and stride: thread (layer group tid/128, token
// tid%TOK), one element per load.
template <typename SCT, int TOK>
__global__ void __launch_bounds__(KT) keep_generic_kernel(KeepArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lvals[];  // [L][TOK]
  const int r = blockIdx.y;
  const int S = min(max(a.seq_used[r], 0), a.max_seq);
  const int t0 = blockIdx.x * TOK;
  if (t0 >= S) return;
  const int tok = threadIdx.x % TOK, lg = threadIdx.x / TOK;
  const int t = t0 + tok;
  const bool body = t < torch_body_end(S);
  if (t < S) {
    const SCT *sbase = (const SCT *)a.scores + (int64_t)r * a.s_sr + t;
    for (int l = lg; l < a.L; l += KT / TOK) {
      const SCT *col = sbase + (int64_t)l * a.s_sl;
      float v;
      if (a.head_reduce == ACTKV_REDUCE_MAX) {
        v = (float)col[0];
        for (int hh = 1; hh < a.H; ++hh) v = nanmax(v, (float)col[(int64_t)hh * a.s_sh]);
      } else {
        auto ld = [&](int hh) { return (float)col[(int64_t)hh * a.s_sh]; };
        v = __fdiv_rn(torch_sum(ld, a.H, body), (float)a.H);
      }
      lvals[l * TOK + tok] = v;
    }
  }
  __syncthreads();
  write_keys<TOK>(a, r, S, t0, lvals);
}

// grid R, 1024 threads: pack bool [S] -> bits (zero-padded to whole blocks)
// and count kept tokens.
__global__ void __launch_bounds__(1024) pack_keep_kernel(const uint8_t *keep, int64_t keep_sr,
                                                         const int32_t *seq_used, int BS,
                                                         uint32_t *bits, int64_t bits_sr,
                                                         int32_t *kept_out, int max_seq) {
  __shared__ uint32_t scratch[32];
  const int r = blockIdx.x;
  const int S = min(max(seq_used[r], 0), max_seq);
  const int padded = ((S + BS - 1) / BS) * BS;
  const int nw = (padded + 31) >> 5;
  const uint8_t *krow = keep + (int64_t)r * keep_sr;
  uint32_t *brow = bits + (int64_t)r * bits_sr;
  // a word of 32 tokens comes from two 16-byte loads when the row is 16-byte aligned and the
  // word lies wholly below S: bit i = (byte i != 0), as in the byte loop
  const bool vec = ((uintptr_t)krow & 15) == 0;
  auto bits4 = [](uint32_t x) {   // 4 bytes -> 4 bits, set where the byte is nonzero
    // (b & 0x7f) + 0x7f carries into bit 7 unless the low 7 bits are zero; | b adds b = 0x80
    const uint32_t y = (((x & 0x7f7f7f7fu) + 0x7f7f7f7fu) | x) & 0x80808080u;
    return ((y >> 7) & 1u) | ((y >> 14) & 2u) | ((y >> 21) & 4u) | ((y >> 28) & 8u);
  };
  uint32_t cnt = 0;
  for (int w = threadIdx.x; w < nw; w += blockDim.x) {
    uint32_t word = 0;
    const int t0 = w * 32;
    if (vec && t0 + 32 <= S) {
      const uint4 lo = *(const uint4 *)(krow + t0), hi = *(const uint4 *)(krow + t0 + 16);
      word = bits4(lo.x) | (bits4(lo.y) << 4) | (bits4(lo.z) << 8) | (bits4(lo.w) << 12) |
             (bits4(hi.x) << 16) | (bits4(hi.y) << 20) | (bits4(hi.z) << 24) | (bits4(hi.w) << 28);
    } else {
      for (int i = 0; i < 32; ++i) {
        const int t = t0 + i;
        if (t < S && krow[t]) word |= 1u << i;
      }
    }
    brow[w] = word;
    cnt += __popc(word);
  }
  const uint32_t tot = block_sum_u32(cnt, scratch);
  if (threadIdx.x == 0 && kept_out) kept_out[r] = (int32_t)tot;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace actkv

using namespace actkv;

extern "C" size_t actkv_workspace_size(int kind, int R, int max_seq) {
  if (kind != ACTKV_WS_KEEP_MASK || R < 1 || max_seq < 0) return 0;
  const size_t keys_sr = ((size_t)max_seq + 3) & ~(size_t)3;
  const size_t stats_sr = ((size_t)max_seq + 63) / 64;
  return align256((size_t)R * keys_sr * 4) + align256((size_t)R * stats_sr * 16);
}

// The launches of actkv_keep_mask on a workspace of workspace_bytes bytes.
static int keep_mask_impl(const void *scores, int scores_dtype, int64_t s_sl, int64_t s_sr,
                          int64_t s_sh, int L, int H, int R, const int32_t *seq_used,
                          const int32_t *budget, const int32_t *protected_count,
                          const uint8_t *protected_mask, int64_t pm_sr, int head_reduce,
                          uint8_t *keep, int64_t keep_sr, uint32_t *keep_bits, int64_t bits_sr,
                          int block_size, int max_seq, void *workspace, size_t workspace_bytes,
                          void *stream) {
  if (!scores || !seq_used || !budget || (!keep && !keep_bits) || L < 1 || H < 1 || R < 1 ||
      max_seq < 0 || block_size < 1)
    return ACTKV_ERR_INVALID_ARG;
  if (protected_count && protected_mask) return ACTKV_ERR_INVALID_ARG;
  if (head_reduce != ACTKV_REDUCE_MEAN && head_reduce != ACTKV_REDUCE_MAX)
    return ACTKV_ERR_INVALID_ARG;
  if (dtype_size(scores_dtype) == 0) return ACTKV_ERR_INVALID_ARG;
  if (L > MAX_LAYERS || H >= (1 << 19) || R > 65535) return ACTKV_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < actkv_workspace_size(ACTKV_WS_KEEP_MASK, R, max_seq))
    return ACTKV_ERR_WORKSPACE;
  if (max_seq == 0) return ACTKV_OK;
  hipStream_t st = (hipStream_t)stream;
  KeepArgs a;
  a.scores = scores; a.s_sl = s_sl; a.s_sr = s_sr; a.s_sh = s_sh;
  a.L = L; a.H = H; a.R = R;
  a.seq_used = seq_used; a.budget = budget; a.prot_count = protected_count;
  a.prot_mask = protected_mask; a.pm_sr = pm_sr; a.head_reduce = head_reduce;
  a.keep = keep; a.keep_sr = keep_sr; a.bits = keep_bits; a.bits_sr = bits_sr;
  a.BS = block_size; a.max_seq = max_seq;
  a.keys = (uint32_t *)workspace;
  a.keys_sr = ((int64_t)max_seq + 3) & ~(int64_t)3;
  a.stats = (uint4 *)((unsigned char *)workspace + align256((size_t)R * a.keys_sr * 4));
  a.stats_sr = ((int64_t)max_seq + 63) / 64;

  const bool vec4 = scores_dtype == ACTKV_F32 && ((uintptr_t)scores & 15) == 0 && s_sl % 4 == 0 &&
                    s_sr % 4 == 0 && s_sh % 4 == 0 && (H == 1 || H == 2 || H == 4 || H == 8 || H == 16);
  // [L][TOK] floats of LDS per block: 128 tokens up to 120 layers, 64 beyond
  const bool wide = L <= MAX_LAYERS_WIDE;
  const int tok = wide ? TOK_WIDE : TOK_NARROW;
  const dim3 grid((unsigned)((max_seq + tok - 1) / tok), (unsigned)R);
  const size_t shm = (size_t)L * tok * sizeof(float);
  auto launch = [&](auto tokc) {
    constexpr int TK = decltype(tokc)::value;
    if (vec4) {
      switch (H) {
        case 1: hipLaunchKernelGGL((keep_vec4_kernel<1, TK>), grid, dim3(KT), shm, st, a); break;
        case 2: hipLaunchKernelGGL((keep_vec4_kernel<2, TK>), grid, dim3(KT), shm, st, a); break;
        case 4: hipLaunchKernelGGL((keep_vec4_kernel<4, TK>), grid, dim3(KT), shm, st, a); break;
        case 8: hipLaunchKernelGGL((keep_vec4_kernel<8, TK>), grid, dim3(KT), shm, st, a); break;
        default: hipLaunchKernelGGL((keep_vec4_kernel<16, TK>), grid, dim3(KT), shm, st, a); break;
      }
    } else switch (scores_dtype) {
      case ACTKV_F32: hipLaunchKernelGGL((keep_generic_kernel<float, TK>), grid, dim3(KT), shm, st, a); break;
      case ACTKV_F16: hipLaunchKernelGGL((keep_generic_kernel<_Float16, TK>), grid, dim3(KT), shm, st, a); break;
      default: hipLaunchKernelGGL((keep_generic_kernel<__bf16, TK>), grid, dim3(KT), shm, st, a); break;
    }
  };
  if (wide) launch(std::integral_constant<int, TOK_WIDE>());
  else launch(std::integral_constant<int, TOK_NARROW>());
  int rc = actkv_check_launch();
  if (rc) return rc;
  hipLaunchKernelGGL(keep_select_kernel, dim3(R), dim3(SEL_T), 0, st, a);
  return actkv_check_launch();
}

extern "C" int actkv_keep_mask(const void *scores, int scores_dtype, int64_t s_sl, int64_t s_sr,
                               int64_t s_sh, int L, int H, int R, const int32_t *seq_used,
                               const int32_t *budget, const int32_t *protected_count,
                               const uint8_t *protected_mask, int64_t pm_sr, int head_reduce,
                               uint8_t *keep, int64_t keep_sr, uint32_t *keep_bits,
                               int64_t bits_sr, int block_size, int max_seq, void *workspace,
                               size_t workspace_bytes, void *stream) {
  return keep_mask_impl(scores, scores_dtype, s_sl, s_sr, s_sh, L, H, R, seq_used, budget,
                        protected_count, protected_mask, pm_sr, head_reduce, keep, keep_sr,
                        keep_bits, bits_sr, block_size, max_seq, workspace, workspace_bytes,
                        stream);
}

// ---------------------------------------------------------------- no-allocation variant
// The workspace of actkv_keep_mask_noalloc: one array per GPU, part of the library's device
// code object, so it exists from module load until the process ends and no call allocates.
// Its host-side name is a stand-in, not a device address: host code uses only the address
// hipGetSymbolAddress returns for the current device, looked up once per device.
static __device__ __align__(256) unsigned char scratch[ACTKV_KEEP_MASK_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
void *scratch_dev[MAX_DEVICES];

int scratch_address(void **out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return ACTKV_ERR_LAUNCH;
  if (dev < 0 || dev >= MAX_DEVICES) return ACTKV_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_dev[dev]) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return ACTKV_ERR_LAUNCH;
    scratch_dev[dev] = p;
  }
  *out = scratch_dev[dev];
  return ACTKV_OK;
}
}  // namespace

extern "C" int actkv_keep_mask_noalloc(const void *scores, int scores_dtype, int64_t s_sl,
                                       int64_t s_sr, int64_t s_sh, int L, int H, int R,
                                       const int32_t *seq_used, const int32_t *budget,
                                       const int32_t *protected_count,
                                       const uint8_t *protected_mask, int64_t pm_sr,
                                       int head_reduce, uint8_t *keep, int64_t keep_sr,
                                       uint32_t *keep_bits, int64_t bits_sr, int block_size,
                                       int max_seq, void *stream) {
  if (R < 1 || max_seq < 0) return ACTKV_ERR_INVALID_ARG;
  if (actkv_workspace_size(ACTKV_WS_KEEP_MASK, R, max_seq) > ACTKV_KEEP_MASK_SCRATCH_BYTES)
    return ACTKV_ERR_WORKSPACE;
  void *ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc) return rc;
  return keep_mask_impl(scores, scores_dtype, s_sl, s_sr, s_sh, L, H, R, seq_used, budget,
                        protected_count, protected_mask, pm_sr, head_reduce, keep, keep_sr,
                        keep_bits, bits_sr, block_size, max_seq, ws,
                        ACTKV_KEEP_MASK_SCRATCH_BYTES, stream);
}

extern "C" int actkv_pack_keep(const uint8_t *keep, int64_t keep_sr, int R, const int32_t *seq_used,
                               int block_size, uint32_t *keep_bits, int64_t bits_sr,
                               int32_t *kept_out, int max_seq, void *stream) {
  if (!keep || !seq_used || !keep_bits || R < 1 || block_size < 1 || max_seq < 0)
    return ACTKV_ERR_INVALID_ARG;
  hipLaunchKernelGGL(pack_keep_kernel, dim3(R), dim3(1024), 0, (hipStream_t)stream, keep, keep_sr,
                     seq_used, block_size, keep_bits, bits_sr, kept_out, max_seq);
  return actkv_check_launch();
}
