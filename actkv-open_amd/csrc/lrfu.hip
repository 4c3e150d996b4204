// LRFU keep-score update (ActKV Algorithm 1 steps 2-4) for the paged cache,
// gfx950.
//
// Reference: actkv/eviction.py:36-50 (top_p_mask) and :209-218
// (ActionLRFU.update_scores), applied to the paged cache's per-token action
// scores.  One workgroup per (layer, request) segment:
//   act[t]  = head reduction (mean in torch's CPU float32 order, or max) of the
//             action-region scores [Hkv, t] for t < seq_used (eviction.py:20-33)
//   hit     = nucleus of act over [protected, seq_used): entries taken in
//             descending order (equal values: lower index first) until the
//             running sum reaches top_p * total, positive entries only
//   ks[t]   = decay * ks[t], then + act[t] where hit (two roundings, as
//             ks.mul_(decay); ks[hit] += a[hit])
// The nucleus is found without sorting: three radix passes (11/11/10 bits of
// the float key) over LDS histograms holding, per bin, the count and the sum
// of the values; walking the bins from the top finds the bin where the running
// sum crosses the threshold, the last pass fixes the exact value, and the tied
// entries at that value are taken in index order.  The bin sums are fixed-point
// integers (each value scaled by 2^(61-E), E the total's exponent), so 64-bit
// integer atomics give the same bits in any order; running sums are compared
// after rounding to float32, as torch's cumsum stores its float64 running sums
// as float32.
#include "common.h"
#include "torch_order.h"

namespace actkv {

constexpr int LT = 1024;        // threads per segment workgroup
constexpr int LB = 2048;        // histogram bins (passes use 2048, 2048, 1024)

struct LrfuArgs {
  const float *scores;
  int64_t s_sl, s_sr, s_sh;
  int L, H, R;
  const int32_t *seq_used, *prot, *active;
  const uint8_t *pmask;  // instead of prot: pinned tokens (excluded, ks untouched)
  int64_t pm_sr;
  float *ks;
  int64_t ks_sl, ks_sr;
  uint8_t *hit;
  int64_t hit_sl, hit_sr;
  float decay, top_p;
  int head_reduce, max_seq;
  float *act;  // workspace [L*R, act_sr]
  int64_t act_sr;
};

// Block sum of doubles (1024 threads).
__device__ double block_sum_f64(double v, double *scratch) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[w] = v;
  __syncthreads();
  double tot = 0.0;
  for (int i = 0; i < LT / 64; ++i) tot += scratch[i];
  __syncthreads();
  return tot;
}

// Walk nb bins from the top (bin nb-1 first) with running sum `base`: find the first
// bin where the running sum, scaled back by qinv and rounded to float32, reaches thr.
// Sums are fixed-point integers (see lrfu_update_kernel), so every order of
// accumulation gives the same bits.  Thread i owns bins nb-1-2i and nb-2-2i.
// Returns the bin (or -1 if the sum never reaches thr); *above = base + sum of the
// bins above it.
typedef unsigned long long u64;
__device__ __forceinline__ float fixed_to_f32(u64 x, double qinv) { return (float)((double)x * qinv); }

__device__ int crossing_bin(const uint32_t *cnt, const u64 *sum, int nb, u64 base, float thr, double qinv,
                            u64 *above, u64 *scratch_q, int *found) {
  const int per = nb / LT;  // 2 or 1
  const int top = nb - 1 - (int)threadIdx.x * per;
  u64 s = 0;
  for (int j = 0; j < per; ++j) s += sum[top - j];
  // inclusive scan over threads in descending-bin order
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  u64 inc = s;
  for (int o = 1; o < 64; o <<= 1) {
    const u64 v = __shfl_up(inc, o, 64);
    if (lane >= o) inc += v;
  }
  if (threadIdx.x == 0) *found = -1;
  __syncthreads();
  if (lane == 63) scratch_q[w] = inc;
  __syncthreads();
  u64 before = base;
  for (int i = 0; i < w; ++i) before += scratch_q[i];
  u64 run = before + inc - s;  // everything above my bins
  for (int j = 0; j < per; ++j) {
    const int b = top - j;
    const u64 next = run + sum[b];
    if (cnt[b] != 0 && fixed_to_f32(run, qinv) < thr && fixed_to_f32(next, qinv) >= thr) {
      *found = b;
      scratch_q[LT / 64] = run;
    }
    run = next;
  }
  __syncthreads();
  const int b = *found;
  if (b >= 0) *above = scratch_q[LT / 64];
  __syncthreads();
  return b;
}

// Per-token action score of a segment: the head reduction (mean in torch's CPU float32
// order, or max) of the scores at token t.
__device__ __forceinline__ float lrfu_head_act(const LrfuArgs &a, const float *sbase, int t, int body_end) {
  const float *col = sbase + t;
  if (a.head_reduce == ACTKV_REDUCE_MAX) {
    float v = col[0];
    for (int hh = 1; hh < a.H; ++hh) v = nanmax(v, col[(int64_t)hh * a.s_sh]);
    return v;
  }
  auto ld = [&](int hh) { return col[(int64_t)hh * a.s_sh]; };
  return __fdiv_rn(torch_sum(ld, a.H, t < body_end), (float)a.H);
}

// grid (ceil(max_seq / 256), L, R), 256 threads: act[t] of every segment's tokens [P, S), one
// token per thread.  It runs ahead of lrfu_update_kernel so that the head reduction's reads
// (Hkv scores per token) are spread over the whole chip instead of one workgroup per segment.
__global__ void __launch_bounds__(256) lrfu_act_kernel(LrfuArgs a) {
  const int l = blockIdx.y, r = blockIdx.z;
  const int S = min(max(a.seq_used[r], 0), a.max_seq);
  const int P = a.prot ? min(max(a.prot[r], 0), S) : 0;
  const int t = P + blockIdx.x * 256 + threadIdx.x;
  if (t >= S) return;
  const float *sbase = a.scores + (int64_t)l * a.s_sl + (int64_t)r * a.s_sr;
  a.act[((int64_t)l * a.R + r) * a.act_sr + t] = lrfu_head_act(a, sbase, t, torch_body_end(S));
}

// grid (L, R), LT threads, after lrfu_act_kernel has written the action scores to the
// workspace.  KMAX > 0: thread i keeps the action scores of its tokens t = P + i + j*LT
// (j < KMAX, segments of up to KMAX*LT tokens) in registers, loaded once with all their
// loads in flight, and every later pass walks the registers (the passes over a workspace
// wait on one load per token in turn); KMAX = 0: every pass reads the workspace (longer
// segments).  Measured on the agent-loop rounds: 91 us against 103 us
// at ~15k tokens with KMAX 16; KMAX 24 (121 registers) took 150 us at ~17k tokens, slower
// than the workspace path, and 32 spills.
template <int KMAX>
__global__ void __launch_bounds__(LT) lrfu_update_kernel(LrfuArgs a) {
  constexpr bool REG = KMAX > 0;
  __shared__ uint32_t cnt[LB];
  __shared__ u64 sum[LB];
  __shared__ double scratch_d[LT / 64];
  __shared__ u64 scratch_q[LT / 64 + 1];
  __shared__ uint32_t scratch_u[LT / 64];
  __shared__ int found;
  __shared__ int cut_s;
  const int l = blockIdx.x, r = blockIdx.y;
  const int S = min(max(a.seq_used[r], 0), a.max_seq);
  // protected tokens: a prefix count, or a pinned mask (then the loops start at 0)
  const int P = a.prot ? min(max(a.prot[r], 0), S) : 0;
  const uint8_t *pin = a.pmask ? a.pmask + (int64_t)r * a.pm_sr : nullptr;
  const bool active = a.active ? a.active[r] != 0 : true;
  float *act = a.act + ((int64_t)l * a.R + r) * a.act_sr;
  float *ks = a.ks + (int64_t)l * a.ks_sl + (int64_t)r * a.ks_sr;
  uint8_t *hit = a.hit ? a.hit + (int64_t)l * a.hit_sl + (int64_t)r * a.hit_sr : nullptr;
  const int tid = threadIdx.x;

  // ---- per-token action score (from lrfu_act_kernel) and the float64 total over [P, S)
  float vals[REG ? KMAX : 1];
  double part = 0.0;
  if constexpr (REG) {
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      const int t = P + tid + j * LT;
      vals[j] = t < S ? act[t] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      const int t = P + tid + j * LT;
      if (t < S && (!pin || !pin[t])) part += (double)vals[j];
    }
  } else {
    for (int t = P + tid; t < S; t += LT) {
      const float v = act[t];
      if (!pin || !pin[t]) part += (double)v;
    }
  }
  // f(t, v) for every token of this thread in [P, S)
  auto for_each = [&](auto f) {
    if constexpr (REG) {
#pragma unroll
      for (int j = 0; j < KMAX; ++j) {
        const int t = P + tid + j * LT;
        if (t < S) f(t, vals[j]);
      }
    } else {
      for (int t = P + tid; t < S; t += LT) f(t, act[t]);
    }
  };
  const double total = block_sum_f64(part, scratch_d);  // (its barriers publish act)
  const float total_f = (float)total;
  const float thr = __fmul_rn(a.top_p, total_f);
  // keys: act >= 0 (means of probabilities), so the float bits order the values
  uint32_t kthr = 0xFFFFFFFFu;  // hit: key > kthr, or key == kthr and t < cut
  int cut = 0;
  if (active && S > P && total_f > 0.f) {
    // Bin sums in fixed point: v -> floor(v * 2^(61-E)), E = the total's exponent, so
    // every value and every sum stays below 2^62 and integer atomics add them in any
    // order to the same bits (float64 atomics would round differently per order).
    // Values below 2^(E-61) count as 0 in the sums; a sum is off by at most one unit per
    // value, under 2^-46 of the total at 32k tokens, far below float32's 2^-24 at thr.
    const int E = ilogb(total);
    const double qscale = ldexp(1.0, 61 - E), qinv = ldexp(1.0, E - 61);
    auto quant = [&](float v) { return (u64)((double)v * qscale); };
    // pass 1: top 11 bits
    for (int b = tid; b < LB; b += LT) { cnt[b] = 0; sum[b] = 0; }
    __syncthreads();
    for_each([&](int t, float v) {
      if (pin && pin[t]) return;
      const uint32_t k = __float_as_uint(v);
      atomicAdd(&cnt[k >> 21], 1u);
      atomicAdd(&sum[k >> 21], quant(v));
    });
    __syncthreads();
    u64 above;
    const int b1 = crossing_bin(cnt, sum, LB, 0, thr, qinv, &above, scratch_q, &found);
    if (b1 < 0) {
      kthr = 0u;          // the sum never reaches the threshold: every positive entry
      cut = 0;
    } else {
      // pass 2: bits [20:10] within bin b1
      for (int b = tid; b < LB; b += LT) { cnt[b] = 0; sum[b] = 0; }
      __syncthreads();
      for_each([&](int t, float v) {
        if (pin && pin[t]) return;
        const uint32_t k = __float_as_uint(v);
        if ((int)(k >> 21) == b1) {
          atomicAdd(&cnt[(k >> 10) & 2047u], 1u);
          atomicAdd(&sum[(k >> 10) & 2047u], quant(v));
        }
      });
      __syncthreads();
      u64 above2;
      int b2 = crossing_bin(cnt, sum, LB, above, thr, qinv, &above2, scratch_q, &found);
      // the sub-bins of b1 add up to b1's sum exactly, so the crossing is found; the
      // fallback (the lowest non-empty bin) only guards the invariant
      if (b2 < 0) {
        b2 = 0;
        for (int b = LB - 1; b >= 0; --b) {
          if (cnt[b]) { b2 = b; }
        }
        u64 run = above;
        for (int b = LB - 1; b > b2; --b) run += sum[b];
        above2 = run;
      }
      // pass 3: bits [9:0] within (b1, b2)
      const uint32_t pre22 = ((uint32_t)b1 << 11) | (uint32_t)b2;
      for (int b = tid; b < LB; b += LT) { cnt[b] = 0; sum[b] = 0; }
      __syncthreads();
      for_each([&](int t, float v) {
        if (pin && pin[t]) return;
        const uint32_t k = __float_as_uint(v);
        if ((k >> 10) == pre22) {
          atomicAdd(&cnt[k & 1023u], 1u);
          atomicAdd(&sum[k & 1023u], quant(v));
        }
      });
      __syncthreads();
      u64 above3;
      int b3 = crossing_bin(cnt, sum, 1024, above2, thr, qinv, &above3, scratch_q, &found);
      if (b3 < 0) {
        b3 = 0;
        for (int b = 1023; b >= 0; --b) {
          if (cnt[b]) { b3 = b; }
        }
        u64 run = above2;
        for (int b = 1023; b > b3; --b) run += sum[b];
        above3 = run;
      }
      kthr = (pre22 << 10) | (uint32_t)b3;
      // ties at the crossing value: the j smallest indices, j = first count at which
      // the running sum, rounded to float32, reaches thr
      const float vstar = __uint_as_float(kthr);
      const u64 qstar = quant(vstar);
      const uint32_t ties = cnt[b3];
      uint32_t need = ties;
      {
        // the running sum with j ties is above3 + j * qstar exactly (integers, and the ties'
        // sum is part of the total, so no overflow), and its float32 rounding never
        // decreases with j: a binary search finds the first j that reaches thr in about
        // log2(ties) steps, where adding one tie at a time took up to S steps when many
        // scores are equal
        auto reached = [&](uint32_t j) { return fixed_to_f32(above3 + (u64)j * qstar, qinv) >= thr; };
        if (ties > 0 && reached(ties)) {
          uint32_t lo = 1, hi = ties;   // reached(hi) holds
          while (lo < hi) {
            const uint32_t mid = lo + (hi - lo) / 2;
            if (reached(mid)) hi = mid;
            else lo = mid + 1;
          }
          need = lo;
        }
      }
      // ordered scan for the index just past the need-th tie: round j covers tokens
      // P + j*LT .. P + j*LT + LT - 1, token P + j*LT + tid being this thread's j-th
      if (tid == 0) cut_s = 0x7fffffff;
      uint32_t running = 0;
      auto scan_round = [&](int j, float v) {
        const int t = P + j * LT + tid;
        const bool f = t < S && !(pin && pin[t]) && __float_as_uint(v) == kthr;
        const unsigned long long bal = __ballot(f);
        const int lane = tid & 63, w = tid >> 6;
        __syncthreads();
        if (lane == 0) scratch_u[w] = (uint32_t)__popcll(bal);
        __syncthreads();
        uint32_t before = running;
        for (int i = 0; i < w; ++i) before += scratch_u[i];
        before += (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
        if (f && before + 1 == need) cut_s = t + 1;
        uint32_t tot = 0;
        for (int i = 0; i < LT / 64; ++i) tot += scratch_u[i];
        running += tot;
        __syncthreads();
      };
      if constexpr (REG) {
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
          if (P + j * LT >= S || running >= need) break;
          scan_round(j, vals[j]);
        }
      } else {
        for (int j = 0; P + j * LT < S && running < need; ++j) {
          const int t = P + j * LT + tid;
          scan_round(j, t < S ? act[t] : 0.f);
        }
      }
      __syncthreads();
      cut = cut_s;
    }
  }
  // ---- keep-score update over [P, S)
  for_each([&](int t, float v) {
    // two roundings, as the reference's ks.mul_(decay) then ks[hit] += act: the compiler
    // must not fuse them into one FMA.  hipcc contracts by default, and the pragma reaches
    // only operations written in this scope (not those inside __fmul_rn / __fadd_rn).
#pragma clang fp contract(off)
    if (pin && pin[t]) {
      if (hit) hit[t] = 0;
      return;
    }
    const uint32_t k = __float_as_uint(v);
    const bool h = v > 0.f && (k > kthr || (k == kthr && t < cut));
    float x = a.decay * ks[t];
    if (h) x = x + v;
    ks[t] = x;
    if (hit) hit[t] = h ? 1 : 0;
  });
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace actkv

using namespace actkv;

extern "C" size_t actkv_lrfu_workspace_size(int L, int R, int max_seq) {
  if (L < 1 || R < 1 || max_seq < 0) return 0;
  return align256((size_t)L * R * (size_t)max_seq * sizeof(float));
}

extern "C" int actkv_lrfu_update(const float *scores, int64_t s_sl, int64_t s_sr, int64_t s_sh, int L,
                                 int H, int R, const int32_t *seq_used, const int32_t *protected_count,
                                 const uint8_t *protected_mask, int64_t pm_sr,
                                 const int32_t *active, float *ks, int64_t ks_sl, int64_t ks_sr,
                                 uint8_t *hit_out, int64_t hit_sl, int64_t hit_sr, float decay,
                                 float top_p, int head_reduce, int max_seq, void *workspace,
                                 size_t workspace_bytes, void *stream) {
  if (!scores || !seq_used || !ks || L < 1 || H < 1 || R < 1 || max_seq < 0)
    return ACTKV_ERR_INVALID_ARG;
  if (head_reduce != ACTKV_REDUCE_MEAN && head_reduce != ACTKV_REDUCE_MAX) return ACTKV_ERR_INVALID_ARG;
  if (protected_count && protected_mask) return ACTKV_ERR_INVALID_ARG;
  if (!(top_p >= 0.f) || !(decay == decay)) return ACTKV_ERR_INVALID_ARG;
  if (L > 65535 || R > 65535) return ACTKV_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < actkv_lrfu_workspace_size(L, R, max_seq)) return ACTKV_ERR_WORKSPACE;
  if (max_seq == 0) return ACTKV_OK;
  LrfuArgs a;
  a.scores = scores; a.s_sl = s_sl; a.s_sr = s_sr; a.s_sh = s_sh;
  a.L = L; a.H = H; a.R = R;
  a.seq_used = seq_used; a.prot = protected_count; a.active = active;
  a.pmask = protected_mask; a.pm_sr = pm_sr;
  a.ks = ks; a.ks_sl = ks_sl; a.ks_sr = ks_sr;
  a.hit = hit_out; a.hit_sl = hit_sl; a.hit_sr = hit_sr;
  a.decay = decay; a.top_p = top_p; a.head_reduce = head_reduce; a.max_seq = max_seq;
  a.act = (float *)workspace; a.act_sr = max_seq;
  // tokens per segment past the protected prefix are at most max_seq
  const dim3 grid(L, R);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(lrfu_act_kernel, dim3((max_seq + 255) / 256, L, R), dim3(256), 0, st, a);
  int rc = actkv_check_launch();
  if (rc) return rc;
  if (max_seq <= 16 * LT) hipLaunchKernelGGL(lrfu_update_kernel<16>, grid, dim3(LT), 0, st, a);
  else hipLaunchKernelGGL(lrfu_update_kernel<0>, grid, dim3(LT), 0, st, a);
  return actkv_check_launch();
}
