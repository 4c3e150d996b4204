// Scores -> keep mask (protected tokens + top-`budget` others) for gfx950.
//
// Reference: actkv/paged.py:23-46 (keep_mask_from_scores).  Three launches,
// batched over requests:
//   keep_reduce : per token, reduce KV heads (mean|max) then average layers,
//                 with the float32 order of torch's CPU `mean` so s[t] is
//                 bit-identical to the reference; write an order-preserving
//                 uint32 key per token (0 marks a protected token) and a
//                 2048-bin histogram of the keys' top 11 bits.
//   keep_select : one workgroup per request finds the exact k-th largest key
//                 with two more 11/10-bit radix passes over the keys, and the
//                 index cut among tied keys (lower index wins).
//   keep_write  : keep[t] = protected | key > thr | (key == thr & t < cut),
//                 also packed LSB-first into 32-bit words for actkv_compact.
//
// torch CPU sum order (aten SumKernel cascade_sum, pinned by the oracle tests):
// for a reduction over n rows of a column block, the column's value is a
// cascade of 16-row blocks (level_power 4) when the column lies in the
// vectorized body (torch_body_end), and the "row_sum" 4-way interleaved order
// for the other columns.  Division by the row count is IEEE (div_, not a
// reciprocal multiply).
#include "common.h"
#include "torch_order.h"

#include <mutex>

namespace actkv {

constexpr int HIST_BINS = 2048;


struct KeepArgs {
  const void *scores;
  int64_t s_sl, s_sr, s_sh;
  int L, H, R;
  const int32_t *seq_used, *budget, *prot_count;
  const uint8_t *prot_mask;
  int64_t pm_sr;
  int head_reduce;
  uint8_t *keep;
  int64_t keep_sr;
  uint32_t *bits;
  int64_t bits_sr;
  int BS, max_seq;
  uint32_t *keys;   // [R, keys_sr], keys_sr = max_seq rounded up to a multiple of 4
  int64_t keys_sr;
  uint32_t *hist;   // [R, HIST_BINS]
  int32_t *sel;     // [R, 4]
};

__device__ __forceinline__ bool is_protected(const KeepArgs &a, int r, int t) {
  if (a.prot_mask) return a.prot_mask[(int64_t)r * a.pm_sr + t] != 0;
  if (a.prot_count) return t < a.prot_count[r];
  return false;
}

constexpr int REDUCE_THREADS = 1024;  // 64 tokens x 16 layer groups

// grid (ceil(max_seq/64), R), REDUCE_THREADS threads: token = tid%64, layer group = tid/64.
template <typename ST>
__global__ void __launch_bounds__(REDUCE_THREADS) keep_reduce_kernel(KeepArgs a) {
  extern __shared__ float lvals[];  // [L][64]
  const int r = blockIdx.y;
  const int S = min(a.seq_used[r], a.max_seq);
  const int t0 = blockIdx.x * 64;
  if (t0 >= S) return;
  const int tok = threadIdx.x & 63, lg = threadIdx.x >> 6;
  const int t = t0 + tok;
  const bool body = t < torch_body_end(S);
  const ST *sbase = (const ST *)a.scores + (int64_t)r * a.s_sr;
  if (t < S) {
    for (int l = lg; l < a.L; l += REDUCE_THREADS / 64) {
      const ST *col = sbase + (int64_t)l * a.s_sl + t;
      float v;
      if (a.head_reduce == ACTKV_REDUCE_MAX) {
        v = (float)col[0];
        for (int hh = 1; hh < a.H; ++hh) v = nanmax(v, (float)col[(int64_t)hh * a.s_sh]);
      } else {
        auto ld = [&](int hh) { return (float)col[(int64_t)hh * a.s_sh]; };
        v = __fdiv_rn(torch_sum(ld, a.H, body), (float)a.H);
      }
      lvals[l * 64 + tok] = v;
    }
  }
  __syncthreads();
  if (threadIdx.x >= 64) return;
  uint32_t key = 0;
  const bool in = t < S;
  if (in && !is_protected(a, r, t)) {
    auto ld = [&](int l) { return lvals[l * 64 + tok]; };
    const float s = __fdiv_rn(torch_sum(ld, a.L, body), (float)a.L);
    key = float_key(s);
  }
  if (in) a.keys[(int64_t)r * a.keys_sr + t] = key;
  // wave-aggregated histogram of candidate keys (key != 0)
  uint32_t *hist = a.hist + (int64_t)r * HIST_BINS;
  bool pending = key != 0;
  const int bin = (int)(key >> 21);
  while (true) {
    const unsigned long long act = __ballot(pending);
    if (act == 0ull) break;
    const int leader = __ffsll((long long)act) - 1;
    const int lbin = __shfl(bin, leader, 64);
    const unsigned long long same = __ballot(pending && bin == lbin);
    if ((int)threadIdx.x == leader) atomicAdd(&hist[lbin], (uint32_t)__popcll(same));
    if (pending && bin == lbin) pending = false;
  }
}

// Histogram of candidate keys (key != 0) by their top 11 bits, one atomic per
// distinct bin of the wave.
__device__ __forceinline__ void hist_add_wave(uint32_t *hist, uint32_t key) {
  bool pending = key != 0;
  const int bin = (int)(key >> 21);
  while (true) {
    const unsigned long long act = __ballot(pending);
    if (act == 0ull) break;
    const int leader = __ffsll((long long)act) - 1;
    const int lbin = __shfl(bin, leader, 64);
    const unsigned long long same = __ballot(pending && bin == lbin);
    if ((int)(threadIdx.x & 63) == leader) atomicAdd(&hist[lbin], (uint32_t)__popcll(same));
    if (pending && bin == lbin) pending = false;
  }
}

// float32 scores with 16-byte aligned token rows: grid (ceil(max_seq/256), R),
// REDUCE_THREADS threads.  Phase 1: thread (layer group tid/64, quad tid%64)
// reduces the heads of 4 consecutive tokens with 16-byte loads; phase 2: each of
// the first 256 threads averages the layers of one token.  Same per-token float
// order as keep_reduce_kernel (a 4-token quad lies wholly in or out of the
// body: torch_body_end is a multiple of 4).
template <int HH>
__global__ void __launch_bounds__(REDUCE_THREADS) keep_reduce4_kernel(KeepArgs a) {
  extern __shared__ float lvals[];  // [L][256]
  const int r = blockIdx.y;
  const int S = min(a.seq_used[r], a.max_seq);
  const int t0 = blockIdx.x * 256;
  if (t0 >= S) return;
  const int quad = threadIdx.x & 63, lg = threadIdx.x >> 6;
  const int tq = t0 + 4 * quad;
  const bool body4 = tq < torch_body_end(S);
  const float *sbase = (const float *)a.scores + (int64_t)r * a.s_sr;
  // the quad's 4 scores of one (layer, head) row; the last quad of a sequence
  // reads only its tokens below S
  const int nin = min(S - tq, 4);
  auto load4 = [&](const float *p) {
    if (nin == 4) return *(const f32x4 *)p;
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < nin; ++j) x[j] = p[j];
    return x;
  };
  if (tq < S) {
    for (int l = lg; l < a.L; l += REDUCE_THREADS / 64) {
      const float *col = sbase + (int64_t)l * a.s_sl + tq;
      f32x4 v;
      if (a.head_reduce == ACTKV_REDUCE_MAX) {
        v = load4(col);
#pragma unroll
        for (int hh = 1; hh < HH; ++hh) {
          const f32x4 x = load4(col + (int64_t)hh * a.s_sh);
          v[0] = nanmax(v[0], x[0]); v[1] = nanmax(v[1], x[1]);
          v[2] = nanmax(v[2], x[2]); v[3] = nanmax(v[3], x[3]);
        }
      } else {
        // the heads of the 4 tokens, loaded once, summed per token
        f32x4 hv[HH];
#pragma unroll
        for (int hh = 0; hh < HH; ++hh) hv[hh] = load4(col + (int64_t)hh * a.s_sh);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          auto ld = [&](int hh) { return hv[hh][j]; };
          v[j] = __fdiv_rn(torch_sum(ld, HH, body4), (float)HH);
        }
      }
      *(f32x4 *)&lvals[l * 256 + 4 * quad] = v;
    }
  }
  __syncthreads();
  if (threadIdx.x >= 256) return;
  const int tok = threadIdx.x;
  const int t = t0 + tok;
  const bool body = t < torch_body_end(S);
  uint32_t key = 0;
  const bool in = t < S;
  if (in && !is_protected(a, r, t)) {
    auto ld = [&](int l) { return lvals[l * 256 + tok]; };
    const float sc = __fdiv_rn(torch_sum(ld, a.L, body), (float)a.L);
    key = float_key(sc);
  }
  if (in) a.keys[(int64_t)r * a.keys_sr + t] = key;
  hist_add_wave(a.hist + (int64_t)r * HIST_BINS, key);
}

// Block-wide helpers for 1024 threads (16 waves).
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

// Find the bin holding the k-th largest element of hist[nbins] (LDS), 1 <= k <=
// total.  Returns the bin; *need = k - (#elements in the bins above it).  Thread
// i owns the nbins/blockDim bins counted from the top; a block-wide exclusive
// scan of those counts (wave shuffles + one LDS pass) lets the one thread whose
// range crosses k resolve the bin.
__device__ int find_bin_desc(const uint32_t *hist, int nbins, uint32_t k, uint32_t *need,
                             uint32_t *scratch) {
  __shared__ int found_bin;
  __shared__ uint32_t found_need;
  const int per = nbins / (int)blockDim.x;          // 2 (2048 bins) or 1 (1024 bins)
  const int top = nbins - 1 - (int)threadIdx.x * per;
  uint32_t c = 0;
  for (int j = 0; j < per; ++j) c += hist[top - j];
  // inclusive wave scan
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t inc = c;
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t v = __shfl_up(inc, o, 64);
    if (lane >= o) inc += v;
  }
  __syncthreads();
  if (lane == 63) scratch[w] = inc;
  __syncthreads();
  uint32_t before = 0;
  for (int i = 0; i < w; ++i) before += scratch[i];
  const uint32_t excl = before + inc - c;          // elements in bins above my range
  if (excl < k && excl + c >= k) {
    uint32_t above = excl;
    int b = top;
    for (int j = 0; j < per; ++j, --b) {
      if (above + hist[b] >= k) break;
      above += hist[b];
    }
    found_bin = b;
    found_need = k - above;
  }
  __syncthreads();
  *need = found_need;
  return found_bin;
}

// Visit keys[0..S) with the whole block: 16-byte loads, four per thread in
// flight before any is used, so a pass costs a few memory latencies, not S/1024.
template <typename F>
__device__ __forceinline__ void scan_keys(const uint32_t *keys, int S, F f) {
  const int S4 = S & ~3;
  const uint4 *k4 = (const uint4 *)keys;  // keys rows are 16-byte aligned (max_seq % 4 == 0)
  constexpr int UNR = 4;
  for (int base = threadIdx.x; base * 4 < S4; base += blockDim.x * UNR) {
    uint4 v[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int i = base + u * blockDim.x;
      v[u] = i * 4 < S4 ? k4[i] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) { f(v[u].x); f(v[u].y); f(v[u].z); f(v[u].w); }
  }
  for (int t = S4 + threadIdx.x; t < S; t += blockDim.x) f(keys[t]);
}

// grid R, 1024 threads.
__global__ void __launch_bounds__(1024) keep_select_kernel(KeepArgs a) {
  __shared__ uint32_t hist[HIST_BINS];
  __shared__ uint32_t scratch[32];
  __shared__ int cut_s;
  const int r = blockIdx.x;
  const int S = min(max(a.seq_used[r], 0), a.max_seq);
  uint32_t *ghist = a.hist + (int64_t)r * HIST_BINS;
  uint32_t local = 0;
  for (int b = threadIdx.x; b < HIST_BINS; b += blockDim.x) {
    const uint32_t v = ghist[b];
    hist[b] = v;
    local += v;
  }
  const uint32_t cand = block_sum_u32(local, scratch);
  const int bud = a.budget[r];
  const uint32_t k = bud <= 0 ? 0u : ((uint32_t)bud < cand ? (uint32_t)bud : cand);
  int32_t *sel = a.sel + (int64_t)r * 4;
  if (k == 0 || k == cand) {
    if (threadIdx.x == 0) {
      sel[0] = k == 0 ? (int32_t)0xFFFFFFFFu : 0;  // keep none / every candidate
      sel[1] = 0;
      sel[2] = (int32_t)cand;
      sel[3] = (int32_t)k;
    }
    return;
  }
  const uint32_t *keys = a.keys + (int64_t)r * a.keys_sr;
  uint32_t need;
  const int b1 = find_bin_desc(hist, HIST_BINS, k, &need, scratch);
  // pass 2: bits [20:10] among keys whose top 11 bits == b1
  for (int b = threadIdx.x; b < HIST_BINS; b += blockDim.x) hist[b] = 0;
  __syncthreads();
  scan_keys(keys, S, [&](uint32_t key) {
    if (key != 0 && (int)(key >> 21) == b1) atomicAdd(&hist[(key >> 10) & 2047u], 1u);
  });
  __syncthreads();
  uint32_t need2;
  const int b2 = find_bin_desc(hist, HIST_BINS, need, &need2, scratch);
  // pass 3: bits [9:0] among keys whose top 22 bits == (b1, b2)
  const uint32_t pre22 = ((uint32_t)b1 << 11) | (uint32_t)b2;
  for (int b = threadIdx.x; b < HIST_BINS; b += blockDim.x) hist[b] = 0;
  __syncthreads();
  scan_keys(keys, S, [&](uint32_t key) {
    if (key != 0 && (key >> 10) == pre22) atomicAdd(&hist[key & 1023u], 1u);
  });
  __syncthreads();
  uint32_t need3;
  const int b3 = find_bin_desc(hist, 1024, need2, &need3, scratch);
  const uint32_t thr = (pre22 << 10) | (uint32_t)b3;
  const uint32_t ties = hist[b3];
  int cut = 0x7fffffff;
  if (need3 < ties) {
    // keep the need3 lowest-index tokens whose key == thr: ordered block scan
    if (threadIdx.x == 0) cut_s = 0x7fffffff;
    uint32_t running = 0;
    for (int base = 0; base < S; base += blockDim.x) {
      const int t = base + threadIdx.x;
      const bool f = t < S && keys[t] == thr;
      const unsigned long long bal = __ballot(f);
      const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
      __syncthreads();
      if (lane == 0) scratch[w] = (uint32_t)__popcll(bal);
      __syncthreads();
      uint32_t before = running;
      for (int i = 0; i < w; ++i) before += scratch[i];
      before += (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
      if (f && before + 1 == need3) cut_s = t + 1;
      uint32_t tot = 0;
      for (int i = 0; i < (int)(blockDim.x >> 6); ++i) tot += scratch[i];
      running += tot;
      __syncthreads();
      if (running >= need3) break;
    }
    __syncthreads();
    cut = cut_s;
  }
  if (threadIdx.x == 0) {
    sel[0] = (int32_t)thr;
    sel[1] = cut;
    sel[2] = (int32_t)cand;
    sel[3] = (int32_t)k;
  }
}

// grid (ceil(max_padded/256), R), 256 threads.
__global__ void __launch_bounds__(256) keep_write_kernel(KeepArgs a) {
  const int r = blockIdx.y;
  const int S = min(max(a.seq_used[r], 0), a.max_seq);
  const int padded = ((S + a.BS - 1) / a.BS) * a.BS;
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (blockIdx.x * 256 >= ((padded + 31) & ~31)) return;
  const int32_t *sel = a.sel + (int64_t)r * 4;
  const uint32_t thr = (uint32_t)sel[0];
  const int cut = sel[1];
  bool kp = false;
  if (t < S) {
    const uint32_t key = a.keys[(int64_t)r * a.keys_sr + t];
    kp = key == 0 || key > thr || (key == thr && t < cut);
    a.keep[(int64_t)r * a.keep_sr + t] = kp ? 1 : 0;
  }
  if (a.bits) {
    const unsigned long long bal = __ballot(kp);
    const int lane = threadIdx.x & 63;
    const int w0 = (t - lane) >> 5;  // word index of lanes 0..31
    const int nw = (padded + 31) >> 5;
    uint32_t *brow = a.bits + (int64_t)r * a.bits_sr;
    if (lane == 0 && w0 < nw) brow[w0] = (uint32_t)(bal & 0xFFFFFFFFull);
    if (lane == 32 && w0 + 1 < nw) brow[w0 + 1] = (uint32_t)(bal >> 32);
  }
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

__global__ void zero_u32_kernel(uint32_t *p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace actkv

using namespace actkv;

extern "C" size_t actkv_workspace_size(int kind, int R, int max_seq) {
  if (kind != ACTKV_WS_KEEP_MASK || R < 1 || max_seq < 0) return 0;
  const size_t keys_sr = ((size_t)max_seq + 3) & ~(size_t)3;
  return align256((size_t)R * keys_sr * 4) + align256((size_t)R * HIST_BINS * 4) +
         align256((size_t)R * 16);
}

// The launches of actkv_keep_mask on a workspace of workspace_bytes bytes.
static int keep_mask_impl(const void *scores, int scores_dtype, int64_t s_sl, int64_t s_sr,
                          int64_t s_sh, int L, int H, int R, const int32_t *seq_used,
                          const int32_t *budget, const int32_t *protected_count,
                          const uint8_t *protected_mask, int64_t pm_sr, int head_reduce,
                          uint8_t *keep, int64_t keep_sr, uint32_t *keep_bits, int64_t bits_sr,
                          int block_size, int max_seq, void *workspace, size_t workspace_bytes,
                          void *stream) {
  if (!scores || !seq_used || !budget || !keep || L < 1 || H < 1 || R < 1 || max_seq < 0 ||
      block_size < 1)
    return ACTKV_ERR_INVALID_ARG;
  if (protected_count && protected_mask) return ACTKV_ERR_INVALID_ARG;
  if (head_reduce != ACTKV_REDUCE_MEAN && head_reduce != ACTKV_REDUCE_MAX)
    return ACTKV_ERR_INVALID_ARG;
  if (dtype_size(scores_dtype) == 0) return ACTKV_ERR_INVALID_ARG;
  if ((size_t)L * 64 * sizeof(float) > 64 * 1024 || H >= (1 << 19)) return ACTKV_ERR_UNSUPPORTED;
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
  unsigned char *ws = (unsigned char *)workspace;
  a.keys_sr = ((int64_t)max_seq + 3) & ~(int64_t)3;
  const size_t keys_bytes = align256((size_t)R * a.keys_sr * 4);
  a.keys = (uint32_t *)ws;
  a.hist = (uint32_t *)(ws + keys_bytes);
  a.sel = (int32_t *)(ws + keys_bytes + align256((size_t)R * HIST_BINS * 4));

  const int64_t nh = (int64_t)R * HIST_BINS;
  hipLaunchKernelGGL(zero_u32_kernel, dim3((unsigned)((nh + 255) / 256)), dim3(256), 0, st, a.hist, nh);
  const bool vec4 = scores_dtype == ACTKV_F32 && ((uintptr_t)scores & 15) == 0 && s_sl % 4 == 0 &&
                    s_sr % 4 == 0 && s_sh % 4 == 0 && (H == 1 || H == 2 || H == 4 || H == 8 || H == 16) &&
                    (size_t)L * 256 * sizeof(float) <= 64 * 1024;
  dim3 g1((max_seq + 63) / 64, R);
  const size_t shm = (size_t)L * 64 * sizeof(float);
  if (vec4) {
    const dim3 g4((max_seq + 255) / 256, R);
    const size_t shm4 = (size_t)L * 256 * sizeof(float);
    switch (H) {
      case 1: hipLaunchKernelGGL(keep_reduce4_kernel<1>, g4, dim3(REDUCE_THREADS), shm4, st, a); break;
      case 2: hipLaunchKernelGGL(keep_reduce4_kernel<2>, g4, dim3(REDUCE_THREADS), shm4, st, a); break;
      case 4: hipLaunchKernelGGL(keep_reduce4_kernel<4>, g4, dim3(REDUCE_THREADS), shm4, st, a); break;
      case 8: hipLaunchKernelGGL(keep_reduce4_kernel<8>, g4, dim3(REDUCE_THREADS), shm4, st, a); break;
      default: hipLaunchKernelGGL(keep_reduce4_kernel<16>, g4, dim3(REDUCE_THREADS), shm4, st, a); break;
    }
  } else switch (scores_dtype) {
    case ACTKV_F32: hipLaunchKernelGGL(keep_reduce_kernel<float>, g1, dim3(REDUCE_THREADS), shm, st, a); break;
    case ACTKV_F16: hipLaunchKernelGGL(keep_reduce_kernel<_Float16>, g1, dim3(REDUCE_THREADS), shm, st, a); break;
    default: hipLaunchKernelGGL(keep_reduce_kernel<__bf16>, g1, dim3(REDUCE_THREADS), shm, st, a); break;
  }
  int rc = actkv_check_launch();
  if (rc) return rc;
  hipLaunchKernelGGL(keep_select_kernel, dim3(R), dim3(1024), 0, st, a);
  if ((rc = actkv_check_launch())) return rc;
  const int64_t padded = ((int64_t)(max_seq + block_size - 1) / block_size) * block_size;
  dim3 g3((unsigned)((padded + 255) / 256), R);
  hipLaunchKernelGGL(keep_write_kernel, g3, dim3(256), 0, st, a);
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
