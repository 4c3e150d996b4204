// Paged attention that emits the softmax log-sum-exp (the lse producer ActKV
// Algorithm 3 consumes) for gfx950.
//
// Reference: actkv/kernels/lse_attn.py:42-60 (paged_decode_attention_ref, the
// stand-in for "the paged FlashAttention backend whose LSE by-product
// Algorithm 3 consumes") and actkv/paged.py:115-118 (decode_attention).  For
// every query row (query n of request r, query head hq) and the tokens t it
// sees (t < seq_used[r], and t < kv_len[r, n] when causal limits are given):
//   s_t = scale * q . k_t,  lse = logsumexp_t s_t,  out = sum_t softmax(s)_t v_t
// out and lse are float32.  A row that sees no token gets lse = -inf, out = 0
// (torch's logsumexp and softmax-einsum over an empty set).
//
// MFMA path (bf16/fp16, head_dim 128, GQA group 1/2/4, more than one 32-row tile of
// query rows per pair): FlashAttention-style,
// one workgroup per (layer, request, KV head, group of NW row tiles), NW waves,
// each owning one 32-row tile of the pair's query rows (n, g) and streaming all
// of the request's tokens.  The transposed products keep every per-query
// quantity inside one lane:
//   S^T = K . Q^T   (v_mfma_f32_32x32x16: A = K rows from LDS, B = Q in registers)
//   lane (lcol, lh) holds s for query row lcol and 16 of the slice's 32 tokens,
//   so the running max / sum of a row are lane-local plus one v_permlane32_swap;
//   O^T += V^T . P^T (A = V^T from LDS, B = P^T: the lane's own 16 probabilities,
//   taken in the token order tau(kb, lh, j) = 16kb + 8(j/4) + 4lh + j%4 that
//   matches the S^T register layout, so no shuffle is needed).
// K and V move through a two-slot LDS stage buffer: the workgroup loads stage
// g+1 into registers while stage g is multiplied, then writes K rows (padded to
// 272 bytes: conflict-free B-operand reads) and V transposed (dim-major rows,
// padded: conflict-free 8-byte reads), one barrier per stage.
//
// Decode path (the same dtypes and shapes when a pair's query rows fit one 32-row
// tile, N*G <= 32): four waves per (pair, token chunk), each streaming its own
// slices through a private LDS region without workgroup barriers; V comes back
// transposed from LDS (ds_read_b64_tr_b16).  Described at attn_decode_kernel.
//
// Generic path (any other dtype / head_dim / group): one workgroup per query row,
// float32 dot products, an online max/sum pass for lse and a second pass that
// accumulates out through LDS-staged probabilities.
#include "common.h"

#include <algorithm>

namespace actkv {

struct AttnArgs {
  const void *q;
  int64_t q_sl, q_sr, q_sn, q_sh;
  const void *kv;  // K plane of layer 0; the V plane is kv + kv_sv elements
  int64_t kv_sl, kv_sv, kv_sb, kv_ss, kv_sh;
  int64_t num_blocks;
  const int32_t *bt;
  int64_t bt_sr;
  int max_blocks;
  const int32_t *seq_used, *n_valid, *kv_len;
  float *out;
  int64_t o_sl, o_sr, o_sn, o_sh;
  float *lse;
  int64_t lse_sl, lse_sr, lse_sn;
  int L, R, N, Hq, Hkv, D, G, BS;
  float scale;
  // token-range split (flash-decoding): chunks per sequence, tokens per chunk, and
  // the partial results of each chunk (row-major [pair][row][chunk])
  int nchunk, tpc, rows_pad;
  float *ws_o;   // [pairs][rows_pad][nchunk][128]: unnormalised sum p v
  float *ws_ml;  // [pairs][rows_pad][nchunk][2]: running max (log2 units), sum p
};

__device__ __forceinline__ int attn_seq_len(const AttnArgs &a, int r) {
  const int s = a.seq_used[r];
  const int span = a.max_blocks * a.BS;
  return s < 0 ? 0 : (s > span ? span : s);
}

__device__ __forceinline__ int attn_nq(const AttnArgs &a, int r) {
  return a.n_valid ? min(max(a.n_valid[r], 0), a.N) : a.N;
}

// tokens query n of request r sees: [0, lim)
__device__ __forceinline__ int attn_lim(const AttnArgs &a, int r, int n, int S) {
  return a.kv_len ? min(max(a.kv_len[(int64_t)r * a.N + n], 0), S) : S;
}

// physical block of logical block `b` of request r, or -1 (past the table, or an
// id outside the pool)
__device__ __forceinline__ int attn_phys(const AttnArgs &a, int r, int b) {
  if (b < 0 || b >= a.max_blocks) return -1;
  const int64_t p = a.bt[(int64_t)r * a.bt_sr + b];
  return (p >= 0 && p < a.num_blocks) ? (int)p : -1;
}

// ------------------------------------------------------------------ MFMA path
template <int NW> struct AttnShape {
  static constexpr int ST = NW >= 4 ? 16 * NW : 32;  // tokens per stage
  static constexpr int GS = ST / 32;                  // 32-token slices per stage
  // a thread stages (4-token group, 16-byte chunk) pairs: 4 K rows and 4 V rows of one chunk
  static constexpr int PPT = (ST / 4) * 16 / (NW * 64);
  static constexpr int KROW = 272;                    // padded K row (bytes)
  // V stage: [token group][dim][4 tokens], 8 bytes per (group, dim)
  static constexpr int KSTAGE = ST * KROW, VSTAGE = ST * 128 * 2;
  static_assert(PPT >= 1 && (ST / 4) * 16 % (NW * 64) == 0, "whole pairs per thread");
};

template <typename T, typename V8, int G, int NW, bool CAUSAL>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW >= 2 ? 2 : 1, NW >= 2 ? 2 : 1)))
attn_mfma_kernel(AttnArgs a, int pairs, int ngroups, int bs_shift) {
  // work item = (pair, row group, token chunk)
  using SH = AttnShape<NW>;
  constexpr int ST = SH::ST, GS = SH::GS, PPT = SH::PPT, KROW = SH::KROW;
  constexpr int KS = 8;
  __shared__ __attribute__((aligned(16))) unsigned char kbuf[2][SH::KSTAGE];
  __shared__ __attribute__((aligned(16))) unsigned char vbuf[2][SH::VSTAGE];

  // XCD-aware mapping: the row groups of one (layer, request, head) pair share an
  // XCD, so the second group's K/V reads hit that XCD's L2.
  const int bid = blockIdx.x;
  const int xcd = bid & 7, jj = bid >> 3;
  const int per_pair = ngroups * a.nchunk;
  const int p = (jj / per_pair) * 8 + xcd;
  const int grp = (jj % per_pair) / a.nchunk, chunk = jj % a.nchunk;
  if (p >= pairs) return;
  const int h = p % a.Hkv;
  const int r = (p / a.Hkv) % a.R;
  const int l = p / (a.Hkv * a.R);
  const int nq = attn_nq(a, r);
  if (grp * NW * 32 >= nq * G) return;
  const int S_all = attn_seq_len(a, r);
  // chunks past the sequence hold nothing the combine step reads
  if (a.nchunk > 1 && chunk * a.tpc >= S_all) return;
  const int c_begin = min(chunk * a.tpc, S_all);
  // this chunk's tokens are [c_begin, c_begin + S); token indices below are relative
  const int S = min(S_all - c_begin, a.tpc);
  const int BS = a.BS;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lcol = lane & 31, lh = lane >> 5;

  // ---- this lane's query row: B operands of S^T = K . Q^T, causal limit
  const int row = (grp * NW + wave) * 32 + lcol;
  const int n = row / G, g = row % G;
  const bool valid = n < nq;
  // tokens of this chunk the row sees: [0, lim) relative to the chunk
  const int lim = valid ? min(max(attn_lim(a, r, n, S_all) - c_begin, 0), S) : 0;
  // the masking limit: padding rows (never written) see everything, so they never force it
  const int lim_m = valid ? lim : 0x7fffffff;
  V8 qf[KS];
  {
    const T *qp = (const T *)a.q + (int64_t)l * a.q_sl + (int64_t)r * a.q_sr +
                  (int64_t)(valid ? n : 0) * a.q_sn + (int64_t)(h * G + g) * a.q_sh + lh * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = *(const V8 *)(qp + ks * 16);
    if (!valid) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qf[ks] = V8{};
    }
  }

  // ---- stage loads: pair q = tid + k*NW*64 of a stage is token group q/16 (tokens
  // 4(q/16) .. +3, one block: groups never straddle a block of >= 16 tokens) and 16-byte
  // chunk q%16 (dims 8(q%16) .. +7)
  const T *kplane = (const T *)a.kv + (int64_t)l * a.kv_sl + (int64_t)h * a.kv_sh;
  const T *vplane = kplane + a.kv_sv;
  // stages up to the furthest token any row of the workgroup sees: a causal prefill's
  // early row groups stop where their queries do instead of masking the rest
  int s_end = S;
  if constexpr (CAUSAL) {
    __shared__ int wg_lim;
    if (tid == 0) wg_lim = 0;
    __syncthreads();
    if (valid && lim > 0) atomicMax(&wg_lim, lim);
    __syncthreads();
    s_end = wg_lim;
  }
  const int nst = (s_end + ST - 1) / ST;
  int phys[PPT];  // physical block of each of this thread's token groups of the next stage
  auto stage_phys = [&](int (&ph)[PPT], int g0) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int t = g0 * ST + 4 * ((tid + k * NW * 64) >> 4);
      ph[k] = t < S ? attn_phys(a, r, (c_begin + t) >> bs_shift) : -1;
    }
  };
  uint4 kreg[PPT][4], vreg[PPT][4];
  auto load_stage = [&](const int (&ph)[PPT], int g0) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int q = tid + k * NW * 64;
      const int t4 = g0 * ST + 4 * (q >> 4), c = q & 15;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t4 + i;
        const bool ok = ph[k] >= 0 && t < S;  // a token of the chunk in a valid block
        const int64_t off = ok ? (int64_t)ph[k] * a.kv_sb + (int64_t)((c_begin + t) & (BS - 1)) * a.kv_ss + c * 8 : 0;
        kreg[k][i] = *(const uint4 *)(kplane + off);
        vreg[k][i] = *(const uint4 *)(vplane + off);
        if (!ok) { kreg[k][i] = make_uint4(0, 0, 0, 0); vreg[k][i] = make_uint4(0, 0, 0, 0); }
      }
    }
  };
  // K rows as they are (padded rows); V as [group][dim][4 tokens]: the 4x8 block of 16-bit
  // values is transposed in registers and written as four 16-byte stores
  auto store_stage = [&](int slot) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int q = tid + k * NW * 64;
      const int tg = q >> 4, c = q & 15;
#pragma unroll
      for (int i = 0; i < 4; ++i) *(uint4 *)(&kbuf[slot][(4 * tg + i) * KROW + c * 16]) = kreg[k][i];
      unsigned char *vd = &vbuf[slot][(tg * 128 + 8 * c) * 8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {  // dims 8c + 2j and 8c + 2j + 1
        auto word = [j](const uint4 &v) { return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w; };
        const uint32_t w0 = word(vreg[k][0]), w1 = word(vreg[k][1]);
        const uint32_t w2 = word(vreg[k][2]), w3 = word(vreg[k][3]);
        uint4 o;
        o.x = (w0 & 0xffffu) | (w1 << 16);          // dim 2j: tokens 0, 1
        o.y = (w2 & 0xffffu) | (w3 << 16);          //         tokens 2, 3
        o.z = (w0 >> 16) | (w1 & 0xffff0000u);      // dim 2j+1: tokens 0, 1
        o.w = (w2 >> 16) | (w3 & 0xffff0000u);      //           tokens 2, 3
        *(uint4 *)(vd + 16 * j) = o;
      }
    }
  };

  const float c2 = a.scale * 1.4426950408889634f;  // logits in log2 units
  float m2 = -INFINITY, lsum = 0.f;
  f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[dt][e] = 0.f;

  if (nst > 0) {
    stage_phys(phys, 0);
    load_stage(phys, 0);
    stage_phys(phys, 1);
    store_stage(0);
  }
  __syncthreads();
  for (int gs = 0; gs < nst; ++gs) {
    const int slot = gs & 1;
    // stage gs+1 into registers (past the end: zero rows, never stored for use)
    load_stage(phys, gs + 1);
    stage_phys(phys, gs + 2);
    // S^T of slice b of this stage: 32 tokens x 32 query rows (dot products, unscaled)
    auto qk = [&](int b) {
      V8 kf[KS];
      const unsigned char *kr = &kbuf[slot][(32 * b + lcol) * KROW + lh * 16];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[ks] = *(const V8 *)(kr + ks * 32);
      f32x16 st = {};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if constexpr (__is_same(T, __bf16))
          st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[ks], st, 0, 0, 0);
        else
          st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[ks], qf[ks], st, 0, 0, 0);
      }
      return st;
    };
    // online softmax of the lane's query row over slice b, then O^T += V^T . P^T
    auto softmax_pv = [&](f32x16 st, int b) {
      const int t0 = gs * ST + 32 * b;
      // tokens at or past a row's limit are masked; slices every row sees whole skip this
      if (__builtin_amdgcn_ballot_w64(lim_m < t0 + 32) != 0ull) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int t = t0 + 8 * (e >> 2) + 4 * lh + (e & 3);
          st[e] = t < lim_m ? st[e] : -INFINITY;
        }
      }
      float mx = st[0];
#pragma unroll
      for (int e = 1; e < 16; ++e) mx = fmaxf(mx, st[e]);
      {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
        mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      }
      const float m_new = fmaxf(m2, mx * c2);  // log2 units (c2 > 0)
      const float msafe = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m2 - msafe);
      float ps = 0.f;
      V8 pb[2];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pe = __builtin_amdgcn_exp2f(fmaf(st[e], c2, -msafe));
        ps += pe;
        pb[e >> 3][e & 7] = (T)pe;
      }
      {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ps), __float_as_uint(ps), false, false);
        ps = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
      }
      lsum = lsum * alpha + ps;
      m2 = m_new;
      // O is rescaled only when some row of the wave raised its max (alpha < 1); the
      // running max settles after the first slices, so most slices skip the 64 multiplies
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0ull) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) oacc[dt][e] *= alpha;
      }
      // O^T += V^T . P^T: A = V^T[32dt + lcol][tau(kb, lh, 0..7)]
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          // tokens 32b + 16kb + 4lh + 0..3 (group g1) and + 8 .. + 11 (group g1 + 2)
          const int g1 = 8 * b + 4 * kb + lh;
          const unsigned char *vr = &vbuf[slot][(g1 * 128 + 32 * dt + lcol) * 8];
          const uint2 lo = *(const uint2 *)vr, hi = *(const uint2 *)(vr + 2 * 128 * 8);
          const uint4 u = make_uint4(lo.x, lo.y, hi.x, hi.y);
          const V8 va = __builtin_bit_cast(V8, u);
          if constexpr (__is_same(T, __bf16))
            oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[kb], oacc[dt], 0, 0, 0);
          else
            oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[kb], oacc[dt], 0, 0, 0);
        }
      }
    };
    // the next slice's S^T chain is issued before this slice's softmax, so the matrix
    // core works while the VALU does the exp/max/sum
    f32x16 st_cur = qk(0);
#pragma unroll
    for (int b = 0; b < GS; ++b) {
      f32x16 st_next = {};
      if (b + 1 < GS) st_next = qk(b + 1);
      softmax_pv(st_cur, b);
      st_cur = st_next;
    }
    if (gs + 1 < nst) store_stage(slot ^ 1);
    __syncthreads();
  }

  // ---- split: the chunk's partial (unnormalised O, max, sum) for the combine kernel
  if (a.nchunk > 1) {
    if (valid) {
      const int64_t pr = ((int64_t)p * a.rows_pad + row) * a.nchunk + chunk;
      float *wo = a.ws_o + pr * 128;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f32x4 v;
          v[0] = oacc[dt][4 * i]; v[1] = oacc[dt][4 * i + 1]; v[2] = oacc[dt][4 * i + 2]; v[3] = oacc[dt][4 * i + 3];
          *(f32x4 *)(wo + 32 * dt + 8 * i + 4 * lh) = v;
        }
      if (lh == 0) { a.ws_ml[pr * 2] = m2; a.ws_ml[pr * 2 + 1] = lsum; }
    }
    return;
  }
  // ---- out[dim] = O^T[dim][row] / lsum, lse = ln 2 * (m2 + log2 lsum)
  if (valid) {
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    float *op = a.out + (int64_t)l * a.o_sl + (int64_t)r * a.o_sr + (int64_t)n * a.o_sn + (int64_t)(h * G + g) * a.o_sh;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d0 = 32 * dt + 8 * i + 4 * lh;
        f32x4 v;
        v[0] = oacc[dt][4 * i] * inv; v[1] = oacc[dt][4 * i + 1] * inv;
        v[2] = oacc[dt][4 * i + 2] * inv; v[3] = oacc[dt][4 * i + 3] * inv;
        *(f32x4 *)(op + d0) = v;
      }
    if (lh == 0)
      a.lse[(int64_t)l * a.lse_sl + (int64_t)r * a.lse_sr + (int64_t)n * a.lse_sn + h * G + g] =
          lsum > 0.f ? (m2 + __log2f(lsum)) * 0.6931471805599453f : -INFINITY;
  }
}

// ------------------------------------------------------------------ decode path
// A pair whose query rows fit one 32-row tile (N*G <= 32: decode steps and short
// action regions) gets a workgroup of DW waves per token chunk, each wave streaming
// the chunk's 32-token slices w, w + DW, ... on its own.  The next slice's K and V
// rows are loaded into registers (coalesced 16-byte loads, four token rows per
// instruction) while the current slice is multiplied out of the wave's private LDS
// region, so the loop has no workgroup barrier.  K rows sit in LDS with their 16-byte
// chunks XOR-swizzled by token (conflict-free A-operand reads); V rows are stored the
// same way and read back with ds_read_b64_tr_b16, which hands each lane four
// consecutive tokens of one dim: the V^T operand with no register transpose.  The
// waves' (max, sum, O) merge through LDS at the end.
constexpr int DW = 4;                         // waves per decode workgroup
constexpr int DREG = 2 * 32 * 256;            // LDS bytes per wave: K rows, then V rows

// 16-byte chunk slot of chunk c of token t: distinct over 16 consecutive tokens (K
// reads), and over the 8 chunks four consecutive tokens expose to a transposed V read
__device__ __forceinline__ int dswz(int t) { return 2 * (t & 7) + ((t >> 3) & 1); }

typedef short dv4s __attribute__((ext_vector_type(4)));

template <typename T, typename V8, int G, bool CAUSAL>
__global__ void __launch_bounds__(DW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
attn_decode_kernel(AttnArgs a, int pairs, int bs_shift) {
  __shared__ __attribute__((aligned(16))) unsigned char reg_lds[DW][DREG];
  __shared__ float mrg_ml[DW][32][2];
  __shared__ int wg_lim;
  const int p = blockIdx.x / a.nchunk, chunk = blockIdx.x % a.nchunk;
  if (p >= pairs) return;
  const int h = p % a.Hkv;
  const int r = (p / a.Hkv) % a.R;
  const int l = p / (a.Hkv * a.R);
  const int nq = attn_nq(a, r);
  if (nq * G <= 0) return;
  const int S_all = attn_seq_len(a, r);
  if (a.nchunk > 1 && chunk * a.tpc >= S_all) return;
  const int c_begin = min(chunk * a.tpc, S_all);
  const int S = min(S_all - c_begin, a.tpc);
  const int BS = a.BS;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int lcol = lane & 31, lh = lane >> 5;
  const int row = lcol;
  const int n = row / G, g = row % G;
  const bool valid = n < nq;
  const int lim = valid ? min(max(attn_lim(a, r, n, S_all) - c_begin, 0), S) : 0;
  const int lim_m = valid ? lim : 0x7fffffff;
  int s_end = S;
  if constexpr (CAUSAL) {
    if (tid == 0) wg_lim = 0;
    __syncthreads();
    if (valid && lim > 0) atomicMax(&wg_lim, lim);
    __syncthreads();
    s_end = wg_lim;
  }
  const int nsl = (s_end + 31) / 32;  // slices of the chunk anyone needs

  V8 qf[8];
  {
    const T *qp = (const T *)a.q + (int64_t)l * a.q_sl + (int64_t)r * a.q_sr +
                  (int64_t)(valid ? n : 0) * a.q_sn + (int64_t)(h * G + g) * a.q_sh + lh * 8;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = *(const V8 *)(qp + ks * 16);
    if (!valid) {
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) qf[ks] = V8{};
    }
  }
  const T *kplane = (const T *)a.kv + (int64_t)l * a.kv_sl + (int64_t)h * a.kv_sh;
  const T *vplane = kplane + a.kv_sv;
  unsigned char *kl = reg_lds[wave];
  unsigned char *vl = kl + 32 * 256;

  // block-table entry of token group i (tokens 4i..4i+3) of slice s: lane i < 8 holds it
  auto slice_phys = [&](int s) {
    const int t = s * 32 + 4 * (lane & 7);
    return (s < nsl && t < S) ? attn_phys(a, r, (c_begin + t) >> bs_shift) : -1;
  };
  // lane: token rows 4i + lane/16 (i = 0..7), 16-byte chunk lane%16, of K and V
  uint4 kr[8], vr[8];
  auto load_slice = [&](int s, int ph) {
    const int c = lane & 15;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int pb = __builtin_amdgcn_readlane(ph, i);
      const int t = s * 32 + 4 * i + (lane >> 4);
      const bool ok = pb >= 0 && t < S;
      const int64_t off = ok ? (int64_t)pb * a.kv_sb + (int64_t)((c_begin + t) & (BS - 1)) * a.kv_ss + c * 8 : 0;
      kr[i] = *(const uint4 *)(kplane + off);
      vr[i] = *(const uint4 *)(vplane + off);
      if (!ok) { kr[i] = make_uint4(0, 0, 0, 0); vr[i] = make_uint4(0, 0, 0, 0); }
    }
  };
  auto store_slice = [&]() {
    const int c = lane & 15;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = 4 * i + (lane >> 4);
      const int o = t * 256 + ((c ^ dswz(t)) << 4);
      *(uint4 *)(kl + o) = kr[i];
      *(uint4 *)(vl + o) = vr[i];
    }
  };

  const float c2 = a.scale * 1.4426950408889634f;
  float m2 = -INFINITY, lsum = 0.f;
  f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[dt][e] = 0.f;

  auto compute = [&](int s) {
    // S^T = K . Q^T for the slice's 32 tokens (A: token lcol, dims 16ks + 8lh .. +7)
    f32x16 st = {};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const int c = 2 * ks + lh;
      const V8 kf = *(const V8 *)(kl + lcol * 256 + ((c ^ dswz(lcol)) << 4));
      if constexpr (__is_same(T, __bf16))
        st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], st, 0, 0, 0);
      else
        st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[ks], st, 0, 0, 0);
    }
    const int t0 = s * 32;
    if (__builtin_amdgcn_ballot_w64(lim_m < t0 + 32) != 0ull) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int t = t0 + 8 * (e >> 2) + 4 * lh + (e & 3);
        st[e] = t < lim_m ? st[e] : -INFINITY;
      }
    }
    float mx = st[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) mx = fmaxf(mx, st[e]);
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
    const float m_new = fmaxf(m2, mx * c2);
    const float msafe = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m2 - msafe);
    float ps = 0.f;
    V8 pb[2];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pe = __builtin_amdgcn_exp2f(fmaf(st[e], c2, -msafe));
      ps += pe;
      pb[e >> 3][e & 7] = (T)pe;
    }
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ps), __float_as_uint(ps), false, false);
      ps = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    lsum = lsum * alpha + ps;
    m2 = m_new;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0ull) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[dt][e] *= alpha;
    }
    // O^T += V^T . P^T.  A = V^T[dim][tau(kb, lh, j)]: two transposed reads give tokens
    // 16kb + 4lh + 0..3 and + 8..11 of dim 32dt + 16((lane/16)&1) + lane%16; lane
    // 4j' + q' of each 16-lane group points at token j', dims 4q' .. 4q'+3
    const int jj = (lane & 15) >> 2, qq = lane & 3;
    const int dgrp = 16 * ((lane >> 4) & 1) + 4 * qq;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const int d = 32 * dt + dgrp;
        const int cc = d >> 3, half = (d >> 2) & 1;
        const int t_lo = 16 * kb + 4 * lh + jj, t_hi = t_lo + 8;
        const dv4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (dv4s __attribute__((address_space(3))) *)(vl + t_lo * 256 + ((cc ^ dswz(t_lo)) << 4) + half * 8));
        const dv4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (dv4s __attribute__((address_space(3))) *)(vl + t_hi * 256 + ((cc ^ dswz(t_hi)) << 4) + half * 8));
        // whole-register casts: the 64-bit results become the operand's two halves
        // (inserting the 16-bit elements one by one compiled to a wrong operand)
        const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
        const V8 va = __builtin_bit_cast(V8, make_uint4(l2.x, l2.y, h2.x, h2.y));
        if constexpr (__is_same(T, __bf16))
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[kb], oacc[dt], 0, 0, 0);
        else
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[kb], oacc[dt], 0, 0, 0);
      }
    }
  };

  // ---- the wave's slices: wave, wave + DW, ...; table entries two slices ahead
  int s = wave;
  int ph_next = slice_phys(s + DW);
  if (s < nsl) load_slice(s, slice_phys(s));
  for (; s < nsl; s += DW) {
    store_slice();
    if (s + DW < nsl) load_slice(s + DW, ph_next);
    ph_next = slice_phys(s + 2 * DW);
    compute(s);
  }

  // ---- merge the waves' (max, sum, O) through LDS
  __syncthreads();
  {
    float *om = (float *)reg_lds[wave];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) om[(dt * 16 + e) * 64 + lane] = oacc[dt][e];
    if (lh == 0) { mrg_ml[wave][lcol][0] = m2; mrg_ml[wave][lcol][1] = lsum; }
  }
  __syncthreads();
  if (wave != 0) return;
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < DW; ++w) M = fmaxf(M, mrg_ml[w][lcol][0]);
  const float Ms = M == -INFINITY ? 0.f : M;
  float Lsum = 0.f, wgt[DW];
#pragma unroll
  for (int w = 0; w < DW; ++w) {
    wgt[w] = __builtin_amdgcn_exp2f(mrg_ml[w][lcol][0] - Ms);
    Lsum += wgt[w] * mrg_ml[w][lcol][1];
  }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < DW; ++w) o += wgt[w] * ((const float *)reg_lds[w])[(dt * 16 + e) * 64 + lane];
      oacc[dt][e] = o;
    }
  if (!valid) return;
  if (a.nchunk > 1) {
    const int64_t pr = ((int64_t)p * a.rows_pad + row) * a.nchunk + chunk;
    float *wo = a.ws_o + pr * 128;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4 v;
        v[0] = oacc[dt][4 * i]; v[1] = oacc[dt][4 * i + 1]; v[2] = oacc[dt][4 * i + 2]; v[3] = oacc[dt][4 * i + 3];
        *(f32x4 *)(wo + 32 * dt + 8 * i + 4 * lh) = v;
      }
    if (lh == 0) { a.ws_ml[pr * 2] = M; a.ws_ml[pr * 2 + 1] = Lsum; }
    return;
  }
  const float inv = Lsum > 0.f ? 1.0f / Lsum : 0.f;
  float *op = a.out + (int64_t)l * a.o_sl + (int64_t)r * a.o_sr + (int64_t)n * a.o_sn + (int64_t)(h * G + g) * a.o_sh;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d0 = 32 * dt + 8 * i + 4 * lh;
      f32x4 v;
      v[0] = oacc[dt][4 * i] * inv; v[1] = oacc[dt][4 * i + 1] * inv;
      v[2] = oacc[dt][4 * i + 2] * inv; v[3] = oacc[dt][4 * i + 3] * inv;
      *(f32x4 *)(op + d0) = v;
    }
  if (lh == 0)
    a.lse[(int64_t)l * a.lse_sl + (int64_t)r * a.lse_sr + (int64_t)n * a.lse_sn + h * G + g] =
        Lsum > 0.f ? (M + __log2f(Lsum)) * 0.6931471805599453f : -INFINITY;
}

// ------------------------------------------------------------------ split combine
// grid ceil(pairs*rows_pad/4), 256 threads: one wave per (pair, row), two dims per lane.
//   M = max_c m_c, w_c = 2^(m_c - M), out = sum_c w_c O_c / sum_c w_c l_c,
//   lse = ln 2 * (M + log2 sum_c w_c l_c)
__global__ void __launch_bounds__(256) attn_combine_kernel(AttnArgs a, int pairs) {
  const int64_t id = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (id >= (int64_t)pairs * a.rows_pad) return;
  const int lane = threadIdx.x & 63;
  const int p = (int)(id / a.rows_pad), row = (int)(id % a.rows_pad);
  const int h = p % a.Hkv;
  const int r = (p / a.Hkv) % a.R;
  const int l = p / (a.Hkv * a.R);
  const int n = row / a.G, g = row % a.G;
  if (n >= attn_nq(a, r)) return;
  const float *ml = a.ws_ml + id * a.nchunk * 2;
  const float *wo = a.ws_o + id * a.nchunk * 128;
  // chunks past the sequence were never written: they hold no token of this row
  const int S_all = attn_seq_len(a, r);
  const int nc = min(a.nchunk, (S_all + a.tpc - 1) / a.tpc);
  float M = -INFINITY;
  for (int c = 0; c < nc; ++c) M = fmaxf(M, ml[2 * c]);
  const float Ms = M == -INFINITY ? 0.f : M;
  float Lsum = 0.f, o0 = 0.f, o1 = 0.f;
  for (int c = 0; c < nc; ++c) {
    const float w = __builtin_amdgcn_exp2f(ml[2 * c] - Ms);
    Lsum += w * ml[2 * c + 1];
    o0 += w * wo[c * 128 + lane];
    o1 += w * wo[c * 128 + 64 + lane];
  }
  const float inv = Lsum > 0.f ? 1.0f / Lsum : 0.f;
  float *op = a.out + (int64_t)l * a.o_sl + (int64_t)r * a.o_sr + (int64_t)n * a.o_sn + (int64_t)(h * a.G + g) * a.o_sh;
  op[lane] = o0 * inv;
  op[64 + lane] = o1 * inv;
  if (lane == 0)
    a.lse[(int64_t)l * a.lse_sl + (int64_t)r * a.lse_sr + (int64_t)n * a.lse_sn + h * a.G + g] =
        Lsum > 0.f ? (M + __log2f(Lsum)) * 0.6931471805599453f : -INFINITY;
}

// ------------------------------------------------------------------ generic path
// grid L*R*N*Hq, 256 threads: one query row per workgroup.
template <typename QT, typename KT>
__global__ void __launch_bounds__(256) attn_generic_kernel(AttnArgs a) {
  extern __shared__ float sm[];  // q [D], then p [256]
  float *qs = sm, *ps = sm + a.D;
  __shared__ float red_m[4], red_l[4];
  const int64_t id = blockIdx.x;
  const int hq = (int)(id % a.Hq);
  const int n = (int)((id / a.Hq) % a.N);
  const int r = (int)((id / ((int64_t)a.Hq * a.N)) % a.R);
  const int l = (int)(id / ((int64_t)a.Hq * a.N * a.R));
  if (n >= attn_nq(a, r)) return;
  const int S = attn_seq_len(a, r);
  const int lim = attn_lim(a, r, n, S);
  const int h = hq / a.G, D = a.D, tid = threadIdx.x;
  const QT *qp = (const QT *)a.q + (int64_t)l * a.q_sl + (int64_t)r * a.q_sr + (int64_t)n * a.q_sn + (int64_t)hq * a.q_sh;
  for (int d = tid; d < D; d += 256) qs[d] = (float)qp[d];
  __syncthreads();
  const KT *kplane = (const KT *)a.kv + (int64_t)l * a.kv_sl + (int64_t)h * a.kv_sh;
  const KT *vplane = kplane + a.kv_sv;
  auto row_off = [&](int t) -> int64_t {
    const int ph = attn_phys(a, r, t / a.BS);
    return ph < 0 ? -1 : (int64_t)ph * a.kv_sb + (int64_t)(t % a.BS) * a.kv_ss;
  };
  auto logit = [&](int t) -> float {
    const int64_t off = row_off(t);
    if (off < 0) return -INFINITY;  // a token in a block the table marks invalid
    float s = 0.f;
    for (int d = 0; d < D; ++d) s = fmaf(qs[d], (float)kplane[off + d], s);
    return s * a.scale;
  };
  // pass 1: online max / sum per thread, then over the workgroup
  float m = -INFINITY, sum = 0.f;
  for (int t = tid; t < lim; t += 256) {
    const float x = logit(t);
    if (x == -INFINITY) continue;
    if (x > m) { sum = sum * expf(m - x) + 1.f; m = x; }
    else sum += expf(x - m);
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float mo = __shfl_xor(m, o, 64), so = __shfl_xor(sum, o, 64);
    const float mn = fmaxf(m, mo);
    sum = (m == -INFINITY ? 0.f : sum * expf(m - mn)) + (mo == -INFINITY ? 0.f : so * expf(mo - mn));
    m = mn;
  }
  if ((tid & 63) == 0) { red_m[tid >> 6] = m; red_l[tid >> 6] = sum; }
  __syncthreads();
  float M = -INFINITY;
  for (int w = 0; w < 4; ++w) M = fmaxf(M, red_m[w]);
  float Lsum = 0.f;
  for (int w = 0; w < 4; ++w) Lsum += red_m[w] == -INFINITY ? 0.f : red_l[w] * expf(red_m[w] - M);
  // pass 2: out = sum_t p_t v_t / Lsum, 256 tokens at a time through LDS
  float acc0 = 0.f, acc1 = 0.f;  // dims tid and tid + 256 (D <= 512)
  for (int t0 = 0; t0 < lim; t0 += 256) {
    __syncthreads();
    const int t = t0 + tid;
    float pt = 0.f;
    if (t < lim) {
      const float x = logit(t);
      pt = x == -INFINITY ? 0.f : expf(x - M);
    }
    ps[tid] = pt;
    __syncthreads();
    const int cnt = min(256, lim - t0);
    for (int j = 0; j < cnt; ++j) {
      const float pj = ps[j];
      if (pj == 0.f) continue;
      const int64_t off = row_off(t0 + j);
      if (tid < D) acc0 = fmaf(pj, (float)vplane[off + tid], acc0);
      if (tid + 256 < D) acc1 = fmaf(pj, (float)vplane[off + tid + 256], acc1);
    }
  }
  float *op = a.out + (int64_t)l * a.o_sl + (int64_t)r * a.o_sr + (int64_t)n * a.o_sn + (int64_t)hq * a.o_sh;
  const float inv = Lsum > 0.f ? 1.0f / Lsum : 0.f;
  if (tid < D) op[tid] = acc0 * inv;
  if (tid + 256 < D) op[tid + 256] = acc1 * inv;
  if (tid == 0)
    a.lse[(int64_t)l * a.lse_sl + (int64_t)r * a.lse_sr + (int64_t)n * a.lse_sn + hq] =
        Lsum > 0.f ? M + logf(Lsum) : -INFINITY;
}

// Waves per workgroup for a launch: enough 32-row tiles for the pair's query rows, at most 8.
static int attn_waves(int rtiles) { return rtiles <= 1 ? 1 : rtiles <= 2 ? 2 : rtiles <= 4 ? 4 : 8; }

// Token-range split: enough (pair, row group, chunk) work items for about four rounds of
// resident workgroups (1 per CU at 8 waves, 2 at 4, 4 at 1-2 waves: the LDS stage
// buffers), chunks of at least 256 tokens, a whole number of stages each.
struct AttnSplit { int nchunk, tpc, rows_pad, ngroups; };
static AttnSplit attn_split(int pairs, int N, int G, int span) {
  AttnSplit sp;
  const int rtiles = (N * G + 31) / 32;
  if (rtiles == 1) {
    // decode kernel: DW waves per (pair, chunk), two workgroups per CU; about two rounds
    // of them, each wave taking at least two 32-token slices of its chunk
    sp.ngroups = 1;
    sp.rows_pad = 32;
    const int unit = DW * 32;
    const int64_t want = 2LL * 2 * 256;
    const int nchunk = (int)std::min<int64_t>(std::max<int64_t>(1, (want + pairs - 1) / pairs),
                                              std::max(1, span / (2 * unit)));
    const int tpc = ((span + nchunk - 1) / nchunk + unit - 1) / unit * unit;
    sp.nchunk = (span + tpc - 1) / tpc;
    sp.tpc = tpc;
    if (sp.nchunk <= 1) { sp.nchunk = 1; sp.tpc = std::max(span, 1); }
    return sp;
  }
  const int nw = attn_waves(rtiles);
  const int st = nw >= 4 ? 16 * nw : 32;
  sp.ngroups = (rtiles + nw - 1) / nw;
  sp.rows_pad = sp.ngroups * nw * 32;
  const int per_cu = nw == 8 ? 1 : nw == 4 ? 2 : 4;
  const int64_t items = (int64_t)pairs * sp.ngroups;
  const int64_t want = 4LL * 256 * per_cu;
  int nchunk = (int)std::min<int64_t>(std::max<int64_t>(1, (want + items - 1) / items), std::max(1, span / 256));
  int tpc = ((span + nchunk - 1) / nchunk + st - 1) / st * st;
  tpc = std::max(tpc, st);
  sp.nchunk = (span + tpc - 1) / tpc;
  sp.tpc = tpc;
  if (sp.nchunk <= 1) { sp.nchunk = 1; sp.tpc = std::max(span, 1); }
  return sp;
}

static size_t attn_ws_bytes(int pairs, const AttnSplit &sp) {
  if (sp.nchunk <= 1) return 0;
  return (size_t)pairs * sp.rows_pad * sp.nchunk * (128 + 2) * sizeof(float);
}

template <typename T, typename V8, int G>
static int launch_attn_mfma(AttnArgs a, int bs_shift, void *ws, size_t ws_bytes, hipStream_t st) {
  const int pairs = a.L * a.R * a.Hkv;
  const int rtiles = (a.N * a.G + 31) / 32;
  const bool causal = a.kv_len != nullptr;
  AttnSplit sp = attn_split(pairs, a.N, a.G, a.max_blocks * a.BS);
  const size_t need = attn_ws_bytes(pairs, sp);
  if (sp.nchunk > 1 && (!ws || ws_bytes < need)) {  // no (large enough) workspace: no split
    sp.nchunk = 1;
    sp.tpc = std::max(a.max_blocks * a.BS, 1);
  }
  a.nchunk = sp.nchunk; a.tpc = sp.tpc; a.rows_pad = sp.rows_pad;
  a.ws_o = sp.nchunk > 1 ? (float *)ws : nullptr;
  a.ws_ml = sp.nchunk > 1 ? (float *)((char *)ws + (size_t)pairs * sp.rows_pad * sp.nchunk * 128 * sizeof(float)) : nullptr;
  if (rtiles == 1) {
    const int grid = pairs * sp.nchunk;
    if (causal)
      hipLaunchKernelGGL((attn_decode_kernel<T, V8, G, true>), dim3(grid), dim3(DW * 64), 0, st, a, pairs, bs_shift);
    else
      hipLaunchKernelGGL((attn_decode_kernel<T, V8, G, false>), dim3(grid), dim3(DW * 64), 0, st, a, pairs, bs_shift);
  } else {
#define ACTKV_ATTN(NWV)                                                                            \
  do {                                                                                             \
    const int grid = ((pairs + 7) / 8) * 8 * sp.ngroups * sp.nchunk;                               \
    if (causal)                                                                                    \
      hipLaunchKernelGGL((attn_mfma_kernel<T, V8, G, NWV, true>), dim3(grid), dim3(NWV * 64), 0,   \
                         st, a, pairs, sp.ngroups, bs_shift);                                      \
    else                                                                                           \
      hipLaunchKernelGGL((attn_mfma_kernel<T, V8, G, NWV, false>), dim3(grid), dim3(NWV * 64), 0,  \
                         st, a, pairs, sp.ngroups, bs_shift);                                      \
  } while (0)
  switch (attn_waves(rtiles)) {
    case 2: ACTKV_ATTN(2); break;
    case 4: ACTKV_ATTN(4); break;
    default: ACTKV_ATTN(8); break;
  }
#undef ACTKV_ATTN
  }
  int rc = actkv_check_launch();
  if (rc || sp.nchunk <= 1) return rc;
  const int64_t waves = (int64_t)pairs * sp.rows_pad;
  hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, a, pairs);
  return actkv_check_launch();
}

template <typename QT, typename KT>
static int launch_attn_generic(const AttnArgs &a, hipStream_t st) {
  const int64_t rows = (int64_t)a.L * a.R * a.N * a.Hq;
  if (rows > 0x7fffffffLL) return ACTKV_ERR_UNSUPPORTED;
  const size_t shm = (size_t)(a.D + 256) * sizeof(float);
  hipLaunchKernelGGL((attn_generic_kernel<QT, KT>), dim3((unsigned)rows), dim3(256), shm, st, a);
  return actkv_check_launch();
}

template <typename QT>
static int dispatch_attn_generic(const AttnArgs &a, int kv_dtype, hipStream_t st) {
  switch (kv_dtype) {
    case ACTKV_F32: return launch_attn_generic<QT, float>(a, st);
    case ACTKV_F16: return launch_attn_generic<QT, _Float16>(a, st);
    case ACTKV_BF16: return launch_attn_generic<QT, __bf16>(a, st);
  }
  return ACTKV_ERR_INVALID_ARG;
}

static bool attn_aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace actkv

using namespace actkv;

extern "C" int actkv_paged_attention(
    const void *q, int q_dtype, int64_t q_sl, int64_t q_sr, int64_t q_sn, int64_t q_sh,
    const void *kv, int kv_dtype, int64_t kv_sl, int64_t kv_sv, int64_t kv_sb, int64_t kv_ss,
    int64_t kv_sh, int64_t num_blocks, const int32_t *block_table, int64_t bt_sr, int max_blocks,
    const int32_t *seq_used, const int32_t *n_valid, const int32_t *kv_len, float *out,
    int64_t o_sl, int64_t o_sr, int64_t o_sn, int64_t o_sh, float *lse, int64_t lse_sl,
    int64_t lse_sr, int64_t lse_sn, int L, int R, int N, int Hq, int Hkv, int D, int block_size,
    float scale, void *workspace, size_t workspace_bytes, void *stream) {
  if (!q || !kv || !block_table || !seq_used || !out || !lse) return ACTKV_ERR_INVALID_ARG;
  if (L < 1 || R < 1 || N < 0 || Hq < 1 || Hkv < 1 || D < 1 || block_size < 1 || max_blocks < 1 ||
      num_blocks < 1)
    return ACTKV_ERR_INVALID_ARG;
  if (Hq % Hkv != 0 || !(scale > 0.f)) return ACTKV_ERR_INVALID_ARG;
  if (dtype_size(q_dtype) == 0 || dtype_size(kv_dtype) == 0) return ACTKV_ERR_INVALID_ARG;
  if ((int64_t)max_blocks * block_size > 0x7fffffffLL || D > 512) return ACTKV_ERR_UNSUPPORTED;
  if (N == 0) return ACTKV_OK;
  hipStream_t st = (hipStream_t)stream;
  AttnArgs a;
  a.q = q; a.q_sl = q_sl; a.q_sr = q_sr; a.q_sn = q_sn; a.q_sh = q_sh;
  a.kv = kv; a.kv_sl = kv_sl; a.kv_sv = kv_sv; a.kv_sb = kv_sb; a.kv_ss = kv_ss; a.kv_sh = kv_sh;
  a.num_blocks = num_blocks;
  a.bt = block_table; a.bt_sr = bt_sr; a.max_blocks = max_blocks;
  a.seq_used = seq_used; a.n_valid = n_valid; a.kv_len = kv_len;
  a.out = out; a.o_sl = o_sl; a.o_sr = o_sr; a.o_sn = o_sn; a.o_sh = o_sh;
  a.lse = lse; a.lse_sl = lse_sl; a.lse_sr = lse_sr; a.lse_sn = lse_sn;
  a.L = L; a.R = R; a.N = N; a.Hq = Hq; a.Hkv = Hkv; a.D = D; a.G = Hq / Hkv; a.BS = block_size;
  a.scale = scale;
  a.nchunk = 1; a.tpc = max_blocks * block_size; a.rows_pad = 0; a.ws_o = nullptr; a.ws_ml = nullptr;
  const int G = a.G;
  int bs_shift = -1;
  for (int sh = 4; sh < 31; ++sh)
    if (block_size == (1 << sh)) bs_shift = sh;
  const bool vec_ok = attn_aligned16(q) && attn_aligned16(kv) && attn_aligned16(out) &&
                      q_sl % 8 == 0 && q_sr % 8 == 0 && q_sn % 8 == 0 && q_sh % 8 == 0 &&
                      kv_sl % 8 == 0 && kv_sv % 8 == 0 && kv_sb % 8 == 0 && kv_ss % 8 == 0 &&
                      kv_sh % 8 == 0 && o_sl % 4 == 0 && o_sr % 4 == 0 && o_sn % 4 == 0 && o_sh % 4 == 0;
  const bool mfma_ok = q_dtype == kv_dtype && (kv_dtype == ACTKV_BF16 || kv_dtype == ACTKV_F16) &&
                       D == 128 && (G == 1 || G == 2 || G == 4) && vec_ok && bs_shift >= 0;
  if (mfma_ok) {
    void *ws = workspace;
    const size_t wb = workspace_bytes;
    if (kv_dtype == ACTKV_BF16)
      return G == 4 ? launch_attn_mfma<__bf16, bf16x8, 4>(a, bs_shift, ws, wb, st)
           : G == 2 ? launch_attn_mfma<__bf16, bf16x8, 2>(a, bs_shift, ws, wb, st)
                    : launch_attn_mfma<__bf16, bf16x8, 1>(a, bs_shift, ws, wb, st);
    return G == 4 ? launch_attn_mfma<_Float16, f16x8, 4>(a, bs_shift, ws, wb, st)
         : G == 2 ? launch_attn_mfma<_Float16, f16x8, 2>(a, bs_shift, ws, wb, st)
                  : launch_attn_mfma<_Float16, f16x8, 1>(a, bs_shift, ws, wb, st);
  }
  switch (q_dtype) {
    case ACTKV_F32: return dispatch_attn_generic<float>(a, kv_dtype, st);
    case ACTKV_F16: return dispatch_attn_generic<_Float16>(a, kv_dtype, st);
    default: return dispatch_attn_generic<__bf16>(a, kv_dtype, st);
  }
}

extern "C" size_t actkv_paged_attention_workspace_size(int L, int R, int N, int Hq, int Hkv, int D,
                                                       int max_blocks, int block_size) {
  if (L < 1 || R < 1 || N < 1 || Hkv < 1 || Hq % Hkv != 0 || max_blocks < 1 || block_size < 1) return 0;
  const int G = Hq / Hkv;
  if (D != 128 || !(G == 1 || G == 2 || G == 4)) return 0;  // the float32 path does not split
  if ((int64_t)max_blocks * block_size > 0x7fffffffLL) return 0;
  const int pairs = L * R * Hkv;
  return attn_ws_bytes(pairs, attn_split(pairs, N, G, max_blocks * block_size));
}
