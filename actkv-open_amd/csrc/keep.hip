// Scores -> keep mask (protected tokens + top-`budget` others) for gfx950.
//
// Reference: actkv/paged.py:23-46 (keep_mask_from_scores).  Two launches,
// batched over requests:
//   keys   : grid (ceil(max_seq/128), R), 512 threads.  Per token, reduce KV
//            heads (mean|max) then average layers, with the float32 order of
//            torch's CPU `mean` so s[t] is bit-identical to the reference, and
//            write an order-preserving uint32 key (0 marks a protected token).
//   select : one 1024-thread block per request, its keys in LDS (chunks of
//            32768 tokens beyond that).  Finds the exact k-th
//            largest key by narrowing a window of key values (2048 bins per
//            pass over the candidates' own range, the window's candidates in LDS
//            once they fit), and the index cut among tied keys (lower index
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

namespace actkv {

constexpr int HIST_BINS = 2048;
constexpr int KT = 512;                 // threads per keys block
constexpr int TOK = 128;                // tokens per keys block
constexpr int SEL_T = 1024;             // threads per select block
constexpr int CAND_CAP = 1536;          // window candidates the select block holds in LDS
constexpr int MAX_LAYERS = 120;         // [L][TOK] layer values fit 60 KiB of LDS

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
  constexpr int U = 4;                             // 16-byte loads in flight per thread (in-bounds
                                                   // clamped reads past n4 are not stored)
  for (int i = threadIdx.x; i < n4; i += U * blockDim.x) {
    uint4 v0 = src[i];                                            // i < n4
    uint4 v1 = src[min(i + (int)blockDim.x, n4 - 1)];
    uint4 v2 = src[min(i + 2 * (int)blockDim.x, n4 - 1)];
    uint4 v3 = src[min(i + 3 * (int)blockDim.x, n4 - 1)];
    ((uint4 *)skeys)[i] = v0;
    if (i + (int)blockDim.x < n4) ((uint4 *)skeys)[i + blockDim.x] = v1;
    if (i + 2 * (int)blockDim.x < n4) ((uint4 *)skeys)[i + 2 * blockDim.x] = v2;
    if (i + 3 * (int)blockDim.x < n4) ((uint4 *)skeys)[i + 3 * blockDim.x] = v3;
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

// Bit width of x (0 for x == 0).
__device__ __forceinline__ int bit_width(uint32_t x) { return x ? 32 - __clz(x) : 0; }

// Inclusive scan over a wave.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  const int lane = threadIdx.x & 63;
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  return v;
}

// The bin holding the k-th largest element of hist[nbins] (LDS), 1 <= k <= total,
// in two barriers; *need = k - (elements in the bins above it).  Thread i owns
// nbins/blockDim bins from the top; wave scans and the per-wave totals give each
// thread its exclusive count, and the one thread whose bins cross k resolves the
// bin.  Between the barriers it clears clear[0, nclear) (the next pass's counts).
__device__ int find_bin(const uint32_t *hist, int nbins, uint32_t k, uint32_t *need, uint32_t *wtot,
                        uint32_t *found, uint32_t *clear, int nclear) {
  const int per = nbins / (int)blockDim.x;
  const int top = nbins - 1 - (int)threadIdx.x * per;
  uint32_t c = 0;
  for (int j = 0; j < per; ++j) c += hist[top - j];
  const uint32_t inc = wave_incl_scan(c);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 63) wtot[w] = inc;
  for (int i = threadIdx.x; i < nclear; i += blockDim.x) clear[i] = 0;
  __syncthreads();
  uint32_t before = 0;
  for (int i = 0; i < w; ++i) before += wtot[i];
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
// passes touch only them.  The passes are arranged for few block barriers: the
// next pass's counts are cleared inside the bin search, counters are set before
// the first barrier.
__global__ void __launch_bounds__(SEL_T) keep_select_kernel(KeepArgs a) {
  __shared__ __attribute__((aligned(16))) uint32_t skeys[KCHUNK];
  __shared__ uint32_t hist_a[HIST_BINS], hist_b[HIST_BINS];
  __shared__ uint2 cand[CAND_CAP];
  __shared__ uint32_t red[3][SEL_T / 64], wtot[SEL_T / 64], found[2];
  __shared__ int ncand_s, ntie_s, cut_s;
  const int r = blockIdx.x;
  const int S = min(max(a.seq_used[r], 0), a.max_seq);
  if (S == 0) return;
  const uint32_t *keys = a.keys + (int64_t)r * a.keys_sr;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int b = threadIdx.x; b < HIST_BINS; b += blockDim.x) hist_a[b] = 0;
  if (threadIdx.x == 0) { ncand_s = 0; ntie_s = 0; cut_s = 0x7fffffff; }
  if (S <= KCHUNK) load_chunk(skeys, keys, 0, S);
  // candidates (unprotected tokens): count, smallest and largest key, from the
  // keys kernel's per-64-token figures, reduced in one barrier
  uint32_t cnt = 0, kmin = 0xFFFFFFFFu, kmax = 0;
  const uint4 *st = a.stats + (int64_t)r * a.stats_sr;
  for (int g = threadIdx.x; g < (S + 63) / 64; g += blockDim.x) {
    const uint4 v = st[g];
    cnt += v.x;
    kmin = min(kmin, v.y);
    kmax = max(kmax, v.z);
  }
  for (int o = 32; o > 0; o >>= 1) {
    cnt += __shfl_xor(cnt, o, 64);
    kmin = min(kmin, (uint32_t)__shfl_xor(kmin, o, 64));
    kmax = max(kmax, (uint32_t)__shfl_xor(kmax, o, 64));
  }
  if (lane == 0) { red[0][wv] = cnt; red[1][wv] = kmin; red[2][wv] = kmax; }
  __syncthreads();
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
    while (true) {
      const int sh = max(0, wbits - 11);     // 2048 bins of 2^sh keys
      auto count = [&](uint32_t key, int) {
        const uint32_t d = key - base;
        if (key != 0 && (wbits >= 32 || d < (1u << wbits))) atomicAdd(&cur[d >> sh], 1u);
      };
      if (in_lds) {
        for (int i = threadIdx.x; i < nc; i += blockDim.x) count(cand[i].x, (int)cand[i].y);
      } else {
        visit_keys(skeys, keys, S, count);
      }
      __syncthreads();
      uint32_t need2;
      const int b = find_bin(cur, HIST_BINS, need, &need2, wtot, found, nxt, HIST_BINS);
      in_win = cur[b];
      need = need2;
      base += (uint32_t)b << sh;
      wbits = sh;
      if (sh == 0) break;                    // the bin is one key value: the threshold
      if (!in_lds && in_win <= (uint32_t)CAND_CAP) {
        // gather the window's candidates (key, index) into LDS
        visit_keys(skeys, keys, S, [&](uint32_t key, int t) {
          if (key != 0 && key - base < (1u << wbits)) cand[atomicAdd(&ncand_s, 1)] = make_uint2(key, (uint32_t)t);
        });
        __syncthreads();
        nc = ncand_s;
        in_lds = true;
      }
      uint32_t *tmp = cur; cur = nxt; nxt = tmp;
    }
    thr = base;
    const uint32_t ties = in_win;            // candidates whose key == thr
    cut = 0x7fffffff;
    if (need < ties && in_lds && ties <= (uint32_t)HIST_BINS) {
      // keep the `need` lowest-index tokens whose key == thr: the tied candidates'
      // indices are gathered from LDS and each finds its rank among them
      uint32_t *tie_t = nxt;
      for (int i = threadIdx.x; i < nc; i += blockDim.x)
        if (cand[i].x == thr) tie_t[atomicAdd(&ntie_s, 1)] = cand[i].y;
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
  // write: a thread's 4 consecutive tokens give one nibble of a 32-token word, the
  // word's 8 nibbles sitting in 8 consecutive lanes; four wave ballots (token j of
  // every lane's group) hold them, and the word's first lane interleaves its byte
  // of each ballot into the word
  const int padded = ((S + a.BS - 1) / a.BS) * a.BS;
  const int nw = (padded + 31) >> 5;
  uint8_t *krow = a.keep ? a.keep + (int64_t)r * a.keep_sr : nullptr;
  uint32_t *brow = a.bits ? a.bits + (int64_t)r * a.bits_sr : nullptr;
  for (int c0 = 0; c0 < padded; c0 += KCHUNK) {
    const int n = min(KCHUNK, S - c0);       // keys of the chunk (n <= 0: padding only)
    if (S > KCHUNK) {
      __syncthreads();
      if (n > 0) load_chunk(skeys, keys, c0, n);
      __syncthreads();
    }
    const int groups = (min(KCHUNK, padded - c0) + 3) >> 2;
    auto group = [&](int g) {                // 4-token group g of the chunk
      uint4 v = make_uint4(0, 0, 0, 0);
      if (4 * g + 3 < n) v = ((const uint4 *)skeys)[g];
      else if (4 * g < n) {
        v.x = skeys[4 * g];
        if (4 * g + 1 < n) v.y = skeys[4 * g + 1];
        if (4 * g + 2 < n) v.z = skeys[4 * g + 2];
      }
      return v;
    };
    auto emit = [&](int g, uint4 v) {
      const int t = c0 + 4 * g;
      const uint32_t kk[4] = {v.x, v.y, v.z, v.w};
      unsigned long long bal[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t key = kk[j];
        const bool kp = t + j < S && (key == 0 || key > thr || (key == thr && t + j < cut));
        bal[j] = __ballot(kp);
        if (krow && t + j < S) krow[t + j] = kp ? 1 : 0;
      }
      const int w = t >> 5;
      if (brow && (lane & 7) == 0 && w < nw) {
        const int sh = lane;                 // 8 * (lane / 8): this word's byte of the ballots
        brow[w] = spread4((uint32_t)(bal[0] >> sh)) | (spread4((uint32_t)(bal[1] >> sh)) << 1) |
                  (spread4((uint32_t)(bal[2] >> sh)) << 2) | (spread4((uint32_t)(bal[3] >> sh)) << 3);
      }
    };
    for (int g0 = 0; g0 < groups; g0 += 2 * blockDim.x) {
      const int g = g0 + threadIdx.x, g2 = g + blockDim.x;
      const uint4 v0 = group(g), v1 = group(g2);
      emit(g, v0);
      if (g0 + blockDim.x < groups) emit(g2, v1);   // uniform over the block
    }
  }
}

// The end of every keys block: layer means of its tokens -> keys, and per 64
// tokens (one wave) the candidate count and the smallest and largest candidate
// key, which the select kernel reduces instead of passing over the keys.  lvals
// [L][TOK] holds the head-reduced score of each (layer, token) of the block.
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
  uint32_t mn = c ? key : 0xFFFFFFFFu, mx = key;
  for (int o = 32; o > 0; o >>= 1) {
    mn = min(mn, (uint32_t)__shfl_xor(mn, o, 64));
    mx = max(mx, (uint32_t)__shfl_xor(mx, o, 64));
  }
  const uint32_t n = (uint32_t)__popcll(__ballot(c));
  if ((tok & 63) == 0 && t < S) a.stats[(int64_t)r * a.stats_sr + t / 64] = make_uint4(n, mn, mx, 0u);
}

// float32 scores with 16-byte aligned token rows: thread (layer group tid/32,
// quad tid%32) reduces the HH heads of 4 consecutive tokens with 16-byte loads,
// up to three layers' loads in flight at once.  Same per-token float order as the
// generic kernel (a 4-token quad lies wholly in or out of the torch body:
// torch_body_end is a multiple of 4).
template <int HH>
__global__ void __launch_bounds__(KT) keep_vec4_kernel(KeepArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lvals[];  // [L][TOK]
  const int r = blockIdx.y;
  const int S = min(max(a.seq_used[r], 0), a.max_seq);
  const int t0 = blockIdx.x * TOK;
  if (t0 >= S) return;
  const int quad = threadIdx.x & 31, lg = threadIdx.x >> 5;  // 16 layer groups
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
    for (int l0 = lg; l0 < a.L; l0 += 16 * LIF) {
      f32x4 hv[LIF][HH];
#pragma unroll
      for (int it = 0; it < LIF; ++it) {
        const int l = l0 + 16 * it;
        if (l < a.L) {
#pragma unroll
          for (int hh = 0; hh < HH; ++hh) hv[it][hh] = load4(sbase + (int64_t)l * a.s_sl + (int64_t)hh * a.s_sh);
        }
      }
#pragma unroll
      for (int it = 0; it < LIF; ++it) {
        const int l = l0 + 16 * it;
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
  write_keys(a, r, S, t0, lvals);
}

// Any score dtype, head count and stride: thread (layer group tid/128, token
// tid%128), one element per load.
template <typename SCT>
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
  write_keys(a, r, S, t0, lvals);
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
  uint32_t cnt = 0;
  for (int w = threadIdx.x; w < nw; w += blockDim.x) {
    uint32_t word = 0;
    const int t0 = w * 32;
    for (int i = 0; i < 32; ++i) {
      const int t = t0 + i;
      if (t < S && krow[t]) word |= 1u << i;
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
  const dim3 grid((unsigned)((max_seq + TOK - 1) / TOK), (unsigned)R);
  const size_t shm = (size_t)L * TOK * sizeof(float);
  if (vec4) {
    switch (H) {
      case 1: hipLaunchKernelGGL(keep_vec4_kernel<1>, grid, dim3(KT), shm, st, a); break;
      case 2: hipLaunchKernelGGL(keep_vec4_kernel<2>, grid, dim3(KT), shm, st, a); break;
      case 4: hipLaunchKernelGGL(keep_vec4_kernel<4>, grid, dim3(KT), shm, st, a); break;
      case 8: hipLaunchKernelGGL(keep_vec4_kernel<8>, grid, dim3(KT), shm, st, a); break;
      default: hipLaunchKernelGGL(keep_vec4_kernel<16>, grid, dim3(KT), shm, st, a); break;
    }
  } else switch (scores_dtype) {
    case ACTKV_F32: hipLaunchKernelGGL(keep_generic_kernel<float>, grid, dim3(KT), shm, st, a); break;
    case ACTKV_F16: hipLaunchKernelGGL(keep_generic_kernel<_Float16>, grid, dim3(KT), shm, st, a); break;
    default: hipLaunchKernelGGL(keep_generic_kernel<__bf16>, grid, dim3(KT), shm, st, a); break;
  }
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
