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
// MFMA path (bf16/fp16, head_dim 128 or 64, any GQA group, more than one 32-row tile
// of query rows per pair): FlashAttention-style,
// one workgroup per (layer, request, KV head, group of NW row tiles), NW waves,
// each owning one 32-row tile of the pair's query rows (n, g) and streaming all
// of the request's tokens.  The transposed products keep every per-query
// quantity inside one lane:
//   S^T = K . Q^T   (v_mfma_f32_32x32x16: A = K rows from LDS, B = Q in registers)
//   lane (lcol, lh) holds s for query row lcol and 16 of the slice's 32 tokens,
//   so the running max / sum of a row are lane-local plus one v_permlane32_swap;
//   O^T += V^T . P^T (A = V^T from LDS, B = P^T: the lane's own 16 probabilities,
//   taken in the token order tau(kb, lh, j) = 16kb + 8(j/4) + 4lh + j%4 that
//   matches the S^T register layout, so no shuffle is needed).  P is split into
//   hi = P rounded to the cache dtype and lo = (P - hi) rounded again, and both
//   terms go through the matrix core: P then carries about 16 significant bits
//   (bf16) instead of 8, so out is within ~1e-5 of the float32 softmax @ v.
// K and V stages go straight from HBM into an LDS ring (buffer loads with the LDS
// bit, several stages ahead), rows XOR-swizzled; V is read back transposed
// (ds_read_b64_tr_b16).  Described at attn_ring_kernel.
//
// Decode path (the same dtypes and shapes when a pair's query rows fit one 32-row
// tile, N*G <= 32): four waves per (pair, token chunk), each streaming its own
// slices through a private LDS region without workgroup barriers; V comes back
// transposed from LDS (ds_read_b64_tr_b16).  Described at attn_decode_kernel.
//
// Head dim 64 runs the same kernels with half-length token rows: a 16-byte load
// instruction then moves eight rows instead of four, the rows' eight 16-byte chunks are
// swizzled with their own pattern (dswz), and two 32-dim output tiles replace four.
//
// Generic path (any other dtype / head_dim up to 512 / block size): float32, up to 8
// query rows of one KV head per workgroup (a decode step's GQA group of up to 8 heads
// reads K and V once), one pass with an online max and sum, token chunks merged by the
// same combine launch.  Described at attn_generic_kernel.
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
  // dyn: the decode kernel's interleaved split (attn_dec_chunks); tpc is then unused
  int nchunk, tpc, rows_pad, dyn;
  float *ws_o;   // [pairs][rows_pad][nchunk][D]: unnormalised sum p v
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

// ------------------------------------------------------------------ chunk merge
// One wave merges the nc token chunks of query row `id` (pair * rows_pad + row) and writes
// out and lse, DH / 64 dims per lane:
//   M = max_c m_c, w_c = 2^(m_c - M), out = sum_c w_c O_c / sum_c w_c l_c,
//   lse = ln 2 * (M + log2 sum_c w_c l_c)
// Lane c reads chunk c's (max, sum) for up to 64 chunks at a time (a butterfly max and sum);
// the O rows of the first 16 chunks are loaded in the same round trip (rows past nc are
// never written: their terms are selected away, not multiplied by zero), later ones after.
template <int DH>
__device__ __forceinline__ void attn_merge_row(const AttnArgs &a, int64_t id, int nc, int64_t o_off,
                                               int64_t lse_off, int lane) {
  static_assert(DH == 64 || DH == 128, "head dims");
  constexpr int PRE = 16;
  const float *ml = a.ws_ml + id * a.nchunk * 2;
  const float *wo = a.ws_o + id * a.nchunk * DH;
  float pre0[PRE], pre1[PRE];
#pragma unroll
  for (int j = 0; j < PRE; ++j) {
    const int jc = max(0, min(j, nc - 1));  // an in-bounds row: the workspace holds nchunk >= max(nc, 1)
    pre0[j] = wo[(int64_t)jc * DH + lane];
    if constexpr (DH == 128) pre1[j] = wo[(int64_t)jc * DH + 64 + lane];
  }
  float M = -INFINITY;
  for (int c = lane; c < nc; c += 64) M = fmaxf(M, ml[2 * c]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
  const float Ms = M == -INFINITY ? 0.f : M;
  float Lsum = 0.f, o0 = 0.f, o1 = 0.f;
  for (int c0 = 0; c0 < nc; c0 += 64) {
    const int c = c0 + lane;
    const float w = c < nc ? __builtin_amdgcn_exp2f(ml[2 * c] - Ms) : 0.f;
    float lw = c < nc ? w * ml[2 * c + 1] : 0.f;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) lw += __shfl_xor(lw, o, 64);
    Lsum += lw;
    if (c0 == 0) {
#pragma unroll
      for (int j = 0; j < PRE; ++j) {
        const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j));
        o0 += j < nc ? wj * pre0[j] : 0.f;
        if constexpr (DH == 128) o1 += j < nc ? wj * pre1[j] : 0.f;
      }
    }
    const float *wc = wo + (int64_t)c0 * DH;
    for (int j = c0 == 0 ? PRE : 0; j < min(64, nc - c0); ++j) {
      const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j));
      o0 += wj * wc[j * DH + lane];
      if constexpr (DH == 128) o1 += wj * wc[j * DH + 64 + lane];
    }
  }
  const float inv = Lsum > 0.f ? 1.0f / Lsum : 0.f;
  float *op = a.out + o_off;
  op[lane] = o0 * inv;
  if constexpr (DH == 128) op[64 + lane] = o1 * inv;
  if (lane == 0) a.lse[lse_off] = Lsum > 0.f ? (M + __log2f(Lsum)) * 0.6931471805599453f : -INFINITY;
}

// The same merge for any head dim (the float32 path's chunks): the chunk weights are
// recomputed for each 64-dim slice of the row.
__device__ __forceinline__ void attn_merge_row_any(const AttnArgs &a, int64_t id, int nc, int64_t o_off,
                                                   int64_t lse_off, int lane) {
  const int D = a.D;
  const float *ml = a.ws_ml + id * a.nchunk * 2;
  const float *wo = a.ws_o + id * a.nchunk * D;
  float M = -INFINITY;
  for (int c = lane; c < nc; c += 64) M = fmaxf(M, ml[2 * c]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
  const float Ms = M == -INFINITY ? 0.f : M;
  float Lsum = 0.f;
  for (int c0 = 0; c0 < nc; c0 += 64) {
    const int c = c0 + lane;
    float lw = c < nc ? exp2f(ml[2 * c] - Ms) * ml[2 * c + 1] : 0.f;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) lw += __shfl_xor(lw, o, 64);
    Lsum += lw;
  }
  const float inv = Lsum > 0.f ? 1.0f / Lsum : 0.f;
  float *op = a.out + o_off;
  for (int d0 = 0; d0 < D; d0 += 64) {
    const int d = d0 + lane;
    float o = 0.f;
    if (d < D)
      for (int c = 0; c < nc; ++c) o += exp2f(ml[2 * c] - Ms) * wo[(int64_t)c * D + d];
    if (d < D) op[d] = o * inv;
  }
  if (lane == 0) a.lse[lse_off] = Lsum > 0.f ? (M + __log2f(Lsum)) * 0.6931471805599453f : -INFINITY;
}

// ------------------------------------------------------------------ MFMA path
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
// waves' (max, sum, O) merge through LDS at the end.  The pairs are split into chunks
// (max(8, 1.5 * CUs / pairs), slices interleaved over their waves: attn_split), merged by the
// combine launch; a sequence whose slices fit one chunk is written here directly.
constexpr int DW = 4;                         // waves per decode workgroup

// Token-row geometry at head dim DH (2-byte elements): one KV head's row of a token is PB
// bytes, NC 16-byte chunks (NC = 2^NCS); a 64-lane 16-byte load moves RPI = 2^RPS rows;
// the S^T product takes KS 16-dim steps and O^T has DT 32-dim tiles.
template <int DH> struct RowShape {
  static_assert(DH == 64 || DH == 128, "head dims");
  static constexpr int PB = 2 * DH, NC = PB / 16, NCS = NC == 16 ? 4 : 3;
  static constexpr int RPI = 64 / NC, RPS = 6 - NCS;
  static constexpr int KS = DH / 16, DT = DH / 32;
  static constexpr int DREG = 2 * 32 * PB;    // decode LDS bytes per wave: K rows, then V rows
};

// The decode split (a.dyn): slice s of a pair (tokens 32s .. 32s + 31) goes to wave
// s mod (nchunk * DW), that is wave s mod DW of chunk (s / DW) mod nchunk.  A wave's slices
// depend on the chunk count only (no other request's length is read); every request spreads
// over the chunks in proportion to its length; and nothing depends on the block table's
// width.  Chunks holding slices of a sequence of S tokens:
__device__ __forceinline__ int attn_dec_chunks(const AttnArgs &a, int S) {
  return min(a.nchunk, (((S + 31) >> 5) + DW - 1) / DW);
}

// 16-byte chunk slot of chunk c of token t is c ^ dswz(t).  Distinct bank groups (the
// address's 16-byte unit mod 16), so no LDS bank conflicts, for: 16 consecutive tokens at
// one chunk (K A-operand reads); four consecutive tokens at four consecutive chunks (a
// 32-lane transposed V read: 16 slots); the chunks of one row (row writes).
//   Head dim 128 (16 chunks, a row is 16 units): 4 (t mod 4) + (t / 4 mod 4).  2 (t mod 8)
//   + (t / 8 mod 2) left the transposed V reads 2-way conflicted.
//   Head dim 64 (8 chunks, a row is 8 units, so rows of odd t use units 8-15): 4 (t / 2 mod 2)
//   + (t / 4 mod 4).  Among 16 tokens each parity takes all 8 values; tokens 4m and 4m + 2
//   (and 4m + 1, 4m + 3) differ in bit 2, so four consecutive chunks of them fall in
//   disjoint halves.
template <int DH>
__device__ __forceinline__ int dswz(int t) {
  if constexpr (DH == 128) return 4 * (t & 3) + ((t >> 2) & 3);
  else return 4 * ((t >> 1) & 1) + ((t >> 2) & 3);
}

typedef short dv4s __attribute__((ext_vector_type(4)));

template <typename T, typename V8, int DH, bool CAUSAL>
__global__ void __launch_bounds__(DW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
attn_decode_kernel(AttnArgs a, int pairs, int bs_shift) {
  using RS = RowShape<DH>;
  constexpr int PB = RS::PB, NC = RS::NC, NCS = RS::NCS, RPI = RS::RPI, KS = RS::KS, DT = RS::DT;
  const int G = a.G;   // query heads per KV head: rows (n, g) of a tile are independent
  __shared__ __attribute__((aligned(16))) unsigned char reg_lds[DW][RS::DREG];
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
  // chunks holding slices; with one (or none: chunk 0 then writes the empty result) the
  // workgroup writes the result itself, with more the combine launch merges them
  const int nact = a.nchunk > 1 ? max(attn_dec_chunks(a, S_all), 1) : 1;
  if (chunk >= nact) return;
  const int S = S_all;
  const int BS = a.BS;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int lcol = lane & 31, lh = lane >> 5;
  const int row = lcol;
  const int n = row / G, g = row % G;
  const bool valid = n < nq;
  const int lim = valid ? min(max(attn_lim(a, r, n, S_all), 0), S) : 0;
  const int lim_m = valid ? lim : 0x7fffffff;
  int s_end = S;
  if constexpr (CAUSAL) {
    if (tid == 0) wg_lim = 0;
    __syncthreads();
    if (valid && lim > 0) atomicMax(&wg_lim, lim);
    __syncthreads();
    s_end = wg_lim;
  }
  const int nsl = (s_end + 31) / 32;  // slices of the pair anyone needs

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
  const T *kplane = (const T *)a.kv + (int64_t)l * a.kv_sl + (int64_t)h * a.kv_sh;
  const T *vplane = kplane + a.kv_sv;
  unsigned char *kl = reg_lds[wave];
  unsigned char *vl = kl + 32 * PB;

  // block-table entry of token group i (tokens 4i..4i+3) of slice s: lane i < 8 holds it.
  // Entries past the sequence are read too (bounds-checked by attn_phys): load_slice skips
  // their tokens.
  auto slice_phys = [&](int s) { return attn_phys(a, r, (s * 32 + 4 * (lane & 7)) >> bs_shift); };
  // lane: token rows RPI i + lane/NC (i < 32/RPI), 16-byte chunk lane%NC, of K and V.  The
  // RPI (4 or 8) rows of one load lie in one block (blocks hold at least 16 tokens), the
  // block of token group RPI i / 4.
  constexpr int NI = 32 / RPI;
  uint4 kr[NI], vr[NI];
  auto load_slice = [&](int s, int ph) {
    const int c = lane & (NC - 1);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int pb = __builtin_amdgcn_readlane(ph, i * RPI / 4);
      const int t = s * 32 + RPI * i + (lane >> NCS);
      const bool ok = pb >= 0 && t < S;
      const int64_t off = ok ? (int64_t)pb * a.kv_sb + (int64_t)(t & (BS - 1)) * a.kv_ss + c * 8 : 0;
      kr[i] = *(const uint4 *)(kplane + off);
      vr[i] = *(const uint4 *)(vplane + off);
      if (!ok) { kr[i] = make_uint4(0, 0, 0, 0); vr[i] = make_uint4(0, 0, 0, 0); }
    }
  };
  auto store_slice = [&]() {
    const int c = lane & (NC - 1);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int t = RPI * i + (lane >> NCS);
      const int o = t * PB + ((c ^ dswz<DH>(t)) << 4);
      *(uint4 *)(kl + o) = kr[i];
      *(uint4 *)(vl + o) = vr[i];
    }
  };

  const float c2 = a.scale * 1.4426950408889634f;
  float m2 = -INFINITY, lsum = 0.f;
  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[dt][e] = 0.f;

  auto compute = [&](int s) {
    // S^T = K . Q^T for the slice's 32 tokens (A: token lcol, dims 16ks + 8lh .. +7)
    f32x16 st = {};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int c = 2 * ks + lh;
      const V8 kf = *(const V8 *)(kl + lcol * PB + ((c ^ dswz<DH>(lcol)) << 4));
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
    V8 pb[2], pbl[2];  // P = hi + lo, both in the cache dtype (hi/lo split below)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pe = __builtin_amdgcn_exp2f(fmaf(st[e], c2, -msafe));
      ps += pe;
      const T hi = (T)pe;
      pb[e >> 3][e & 7] = hi;
      pbl[e >> 3][e & 7] = (T)(pe - (float)hi);
    }
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ps), __float_as_uint(ps), false, false);
      ps = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    lsum = lsum * alpha + ps;
    m2 = m_new;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0ull) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
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
      for (int dt = 0; dt < DT; ++dt) {
        const int d = 32 * dt + dgrp;
        const int cc = d >> 3, half = (d >> 2) & 1;
        const int t_lo = 16 * kb + 4 * lh + jj, t_hi = t_lo + 8;
        const dv4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (dv4s __attribute__((address_space(3))) *)(vl + t_lo * PB + ((cc ^ dswz<DH>(t_lo)) << 4) + half * 8));
        const dv4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (dv4s __attribute__((address_space(3))) *)(vl + t_hi * PB + ((cc ^ dswz<DH>(t_hi)) << 4) + half * 8));
        // whole-register casts: the 64-bit results become the operand's two halves
        // (inserting the 16-bit elements one by one compiled to a wrong operand)
        const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
        const V8 va = __builtin_bit_cast(V8, make_uint4(l2.x, l2.y, h2.x, h2.y));
        if constexpr (__is_same(T, __bf16)) {
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[kb], oacc[dt], 0, 0, 0);
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pbl[kb], oacc[dt], 0, 0, 0);
        } else {
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[kb], oacc[dt], 0, 0, 0);
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pbl[kb], oacc[dt], 0, 0, 0);
        }
      }
    }
  };

  // ---- the wave's slices: wave, wave + DW, ...; table entries two slices ahead
  const int step = a.nchunk * DW;
  int s = chunk * DW + wave;
  int ph_next = slice_phys(s + step);
  if (s < nsl) load_slice(s, slice_phys(s));
  for (; s < nsl; s += step) {
    store_slice();
    if (s + step < nsl) load_slice(s + step, ph_next);
    ph_next = slice_phys(s + 2 * step);
    compute(s);
  }

  // ---- merge the waves' (max, sum, O) through LDS
  __syncthreads();
  {
    float *om = (float *)reg_lds[wave];   // DT x 4 KiB: the wave's DREG bytes
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) om[(dt * 16 + e) * 64 + lane] = oacc[dt][e];
    if (lh == 0) { mrg_ml[wave][lcol][0] = m2; mrg_ml[wave][lcol][1] = lsum; }
  }
  __syncthreads();
  if (wave == 0) {
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
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float o = 0.f;
#pragma unroll
        for (int w = 0; w < DW; ++w) o += wgt[w] * ((const float *)reg_lds[w])[(dt * 16 + e) * 64 + lane];
        oacc[dt][e] = o;
      }
    if (valid && nact > 1) {  // this chunk's partial result
      const int64_t pr = ((int64_t)p * a.rows_pad + row) * a.nchunk + chunk;
      float *wo = a.ws_o + pr * DH;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f32x4 v;
          v[0] = oacc[dt][4 * i]; v[1] = oacc[dt][4 * i + 1]; v[2] = oacc[dt][4 * i + 2]; v[3] = oacc[dt][4 * i + 3];
          *(f32x4 *)(wo + 32 * dt + 8 * i + 4 * lh) = v;
        }
      if (lh == 0) { a.ws_ml[pr * 2] = M; a.ws_ml[pr * 2 + 1] = Lsum; }
    } else if (valid) {       // the whole sequence: the result
      const float inv = Lsum > 0.f ? 1.0f / Lsum : 0.f;
      float *op = a.out + (int64_t)l * a.o_sl + (int64_t)r * a.o_sr + (int64_t)n * a.o_sn + (int64_t)(h * G + g) * a.o_sh;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
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
  }
}

// ------------------------------------------------------------------ ring path
// Pairs with more than one 32-row tile.  A workgroup of NW waves (one row tile each)
// shares ST-token stages of K and V held in an NSTG-deep LDS ring.  The stages are
// loaded straight into LDS with buffer_load_dwordx4 ... lds, NSTG - 1 stages ahead of
// the one being multiplied: no register staging, one LDS barrier per stage, and the
// wait for a stage is counted by hand (wait_stages).  Each load instruction moves
// four token rows (eight at head dim 64; 1 KB) of one block, so the buffer resource is that
// block (wave-uniform); its lanes pick the global 16-byte chunk that lands in their LDS
// slot, which lays rows out with the decode path's XOR swizzle, and tokens past the
// chunk (or in blocks the table marks invalid) are out of the resource's range, so the
// hardware writes zeros.  V is read back transposed (ds_read_b64_tr_b16).  The block
// table of the workgroup's token range sits in an LDS window, refilled (after a drain)
// when the loads reach its end.

// s_waitcnt with vmcnt <= N and the other counters unconstrained
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// workgroup barrier ordering LDS only (no drain of the loads in flight)
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Stage size and ring depth, from a sweep on 36 layers x 32k tokens x 128 queries and on
// 4 requests x 8k tokens x 48 causal queries: with the loads issued ahead, depth matters
// little (3 or 4 stages of 64 tokens and 2 of 128 are within 8%) and fewer, larger stages
// (fewer barriers) win; 4- and 2-wave workgroups keep 64-token stages so that two fit
// per CU.
template <int TILES, int DH> struct RingShape {             // TILES: row tiles per workgroup
  static constexpr int ST = TILES >= 8 ? 128 : 64;            // tokens per stage
  static constexpr int NSTG = 2;                              // ring depth
  static constexpr int TBLW = TILES >= 8 ? 4096 : 2048;       // block-table window (entries)
  static constexpr int SBYTES = 2 * ST * RowShape<DH>::PB;    // K then V rows of a stage
  static constexpr int IPP = ST / RowShape<DH>::RPI;          // load instructions per plane
  static_assert(ST % 32 == 0, "whole slices per stage");
};

// wait until at most `rem` stages' loads (PER instructions each) are outstanding
template <int PER, int MAXR>
__device__ __forceinline__ void wait_stages(int rem) {
  if constexpr (MAXR >= 3) { if (rem >= 3) { wait_vmcnt<3 * PER>(); return; } }
  if constexpr (MAXR >= 2) { if (rem >= 2) { wait_vmcnt<2 * PER>(); return; } }
  if constexpr (MAXR >= 1) { if (rem >= 1) { wait_vmcnt<PER>(); return; } }
  wait_vmcnt<0>();
}

typedef int ri32x4 __attribute__((ext_vector_type(4)));

// 16 bytes from buffer `rsrc` at byte offset voff into LDS at lds_base + 16 * lane.
// Inline assembly: the compiler's wait counting would otherwise drain every load in
// flight before each LDS read of the ring; the kernel counts them itself.  M0 carries
// the LDS base and is restored.
__device__ __forceinline__ void buf_lds16(ri32x4 rsrc, unsigned voff, unsigned lds_base) {
  unsigned saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(voff), "s"(rsrc), "s"(lds_base)
               : "memory");
}

template <typename T, typename V8, int DH, int NW, int RT, bool CAUSAL>
__global__ void __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu(RT >= 2 ? 1 : (NW >= 4 ? 2 : 1), RT >= 2 ? 1 : 2)))
attn_ring_kernel(AttnArgs a, int pairs, int ngroups, int bs_shift) {
  const int G = a.G;   // query heads per KV head: rows (n, g) of a tile are independent
  using SH = RingShape<NW * RT, DH>;
  using RS = RowShape<DH>;
  constexpr int PB = RS::PB, NC = RS::NC, NCS = RS::NCS, RPI = RS::RPI, KS = RS::KS, DT = RS::DT;
  constexpr int ST = SH::ST, NSTG = SH::NSTG, TBLW = SH::TBLW;
  constexpr int PER = 2 * SH::IPP / NW;  // load instructions per wave per stage
  static_assert((2 * SH::IPP) % NW == 0, "whole load instructions per wave");
  __shared__ __attribute__((aligned(1024))) unsigned char ring[NSTG][SH::SBYTES];
  __shared__ int tbl[TBLW];
  __shared__ int wg_lim;

  // XCD-aware mapping: the row groups and chunks of one pair share an XCD
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
  if (grp * NW * RT * 32 >= nq * G) return;
  const int S_all = attn_seq_len(a, r);
  if (a.nchunk > 1 && chunk * a.tpc >= S_all) return;
  const int c_begin = min(chunk * a.tpc, S_all);
  const int S = min(S_all - c_begin, a.tpc);
  const int BS = a.BS;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int lcol = lane & 31, lh = lane >> 5;
  // the wave's RT row tiles: rows ((grp * NW + wave) * RT + rt) * 32 + lcol
  int row[RT], n[RT], g[RT], lim_m[RT];
  bool valid[RT];
  int my_lim = 0;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    row[rt] = ((grp * NW + wave) * RT + rt) * 32 + lcol;
    n[rt] = row[rt] / G;
    g[rt] = row[rt] % G;
    valid[rt] = n[rt] < nq;
    const int lim = valid[rt] ? min(max(attn_lim(a, r, n[rt], S_all) - c_begin, 0), S) : 0;
    // the masking limit: padding rows (never written) see everything, so they never force it
    lim_m[rt] = valid[rt] ? lim : 0x7fffffff;
    my_lim = max(my_lim, lim);
  }
  int s_end = S;
  if constexpr (CAUSAL) {
    if (tid == 0) wg_lim = 0;
    __syncthreads();
    if (my_lim > 0) atomicMax(&wg_lim, my_lim);
    __syncthreads();
    s_end = wg_lim;
  }
  const int nst = (s_end + ST - 1) / ST;

  V8 qf[RT][KS];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const T *qp = (const T *)a.q + (int64_t)l * a.q_sl + (int64_t)r * a.q_sr +
                  (int64_t)(valid[rt] ? n[rt] : 0) * a.q_sn + (int64_t)(h * G + g[rt]) * a.q_sh + lh * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[rt][ks] = *(const V8 *)(qp + ks * 16);
    if (!valid[rt]) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qf[rt][ks] = V8{};
    }
  }
  // the query loads complete here, before the first ring load: otherwise the compiler's
  // wait for them lands inside the loop, where the hardware counter also holds the
  // ring's loads and the wait would drain them every stage
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) asm volatile("" ::"v"(qf[rt][ks]));

  // ---- block table window: logical blocks [blk0 + wbase, blk0 + wbase + TBLW)
  const int blk0 = c_begin >> bs_shift;
  int wbase = 0;
  auto load_window = [&]() {
    for (int i = tid; i < TBLW; i += NW * 64) tbl[i] = attn_phys(a, r, blk0 + wbase + i);
  };
  load_window();
  __syncthreads();
  // before issuing stage gi: move the window when the stage's last block is past it (the
  // workgroup calls this uniformly; a stage spans at most ST / BS + 1 blocks)
  auto ensure_window = [&](int gi) {
    const int lb = ((c_begin + gi * ST + ST - 1) >> bs_shift) - blk0;
    if (lb - wbase >= TBLW) {
      __syncthreads();
      wbase = ((c_begin + gi * ST) >> bs_shift) - blk0;
      load_window();
      __syncthreads();
    }
  };

  // ---- stage loads: instruction k of a stage: plane k / IPP, tokens RPI(k % IPP) .. +RPI-1
  const uint64_t kbase = (uint64_t)(uintptr_t)((const T *)a.kv + (int64_t)l * a.kv_sl + (int64_t)h * a.kv_sh);
  const uint64_t vbase = kbase + (uint64_t)a.kv_sv * sizeof(T);
  const unsigned blk_bytes = (unsigned)(((int64_t)(BS - 1) * a.kv_ss + DH) * sizeof(T));
  const unsigned ring_base = (unsigned)(uintptr_t)&ring[0][0];
  auto issue = [&](int gi) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int k = wave * PER + i;
      const int plane = k / SH::IPP, tg = k % SH::IPP;
      const int t0 = gi * ST + RPI * tg;                     // chunk-relative first token
      const int bi = ((c_begin + t0) >> bs_shift) - blk0 - wbase;
      const int ph = __builtin_amdgcn_readfirstlane(tbl[bi]);
      const uint64_t bb = (plane ? vbase : kbase) + (uint64_t)(ph < 0 ? 0 : ph) * (uint64_t)a.kv_sb * sizeof(T);
      ri32x4 rs;
      rs[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)bb);
      rs[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(bb >> 32) & 0xffffu));
      rs[2] = __builtin_amdgcn_readfirstlane(ph < 0 ? 0 : (int)blk_bytes);
      rs[3] = 0x00020000;
      const int tl = RPI * tg + (lane >> NCS);               // token within the stage
      const int t = gi * ST + tl;
      const int c = (lane & (NC - 1)) ^ dswz<DH>(tl);         // global chunk landing in slot lane%NC
      const unsigned voff = t < S ? (unsigned)((((c_begin + t) & (BS - 1)) * a.kv_ss + c * 8) * sizeof(T)) : 0xfffffff0u;
      const unsigned dst = ring_base + (unsigned)((gi % NSTG) * SH::SBYTES + plane * ST * PB + tg * 1024);
      buf_lds16(rs, voff, __builtin_amdgcn_readfirstlane(dst));
    }
  };

  const float c2 = a.scale * 1.4426950408889634f;
  float m2[RT], lsum[RT];
  f32x16 oacc[RT][DT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m2[rt] = -INFINITY;
    lsum[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) oacc[rt][dt][e] = 0.f;
  }

  const int jq = (lane & 15) >> 2, qq = lane & 3;
  const int dgrp = 16 * ((lane >> 4) & 1) + 4 * qq;
  struct Tiles { f32x16 s[RT]; };
  // S^T = K . Q^T of one 32-token slice for every row tile: each K fragment read once
  auto qk = [&](const unsigned char *kl) {
    Tiles st;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) st.s[rt] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int c = 2 * ks + lh;
      const V8 kf = *(const V8 *)(kl + lcol * PB + ((c ^ dswz<DH>(lcol)) << 4));
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        if constexpr (__is_same(T, __bf16))
          st.s[rt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[rt][ks], st.s[rt], 0, 0, 0);
        else
          st.s[rt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[rt][ks], st.s[rt], 0, 0, 0);
      }
    }
    return st;
  };
  // online softmax of each tile's rows over the slice, then O^T += V^T . P^T with each V^T
  // fragment read once for all tiles
  auto softmax_pv = [&](Tiles &st, const unsigned char *vl, int t0) {
    V8 pb[RT][2], pbl[RT][2];  // P = hi + lo, both in the cache dtype
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      f32x16 &x = st.s[rt];
      if (__builtin_amdgcn_ballot_w64(lim_m[rt] < t0 + 32) != 0ull) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int t = t0 + 8 * (e >> 2) + 4 * lh + (e & 3);
          x[e] = t < lim_m[rt] ? x[e] : -INFINITY;
        }
      }
      float mx = x[0];
#pragma unroll
      for (int e = 1; e < 16; ++e) mx = fmaxf(mx, x[e]);
      {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
        mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      }
      const float m_new = fmaxf(m2[rt], mx * c2);
      const float msafe = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m2[rt] - msafe);
      float ps = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pe = __builtin_amdgcn_exp2f(fmaf(x[e], c2, -msafe));
        ps += pe;
        const T hi = (T)pe;
        pb[rt][e >> 3][e & 7] = hi;
        pbl[rt][e >> 3][e & 7] = (T)(pe - (float)hi);
      }
      {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ps), __float_as_uint(ps), false, false);
        ps = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
      }
      lsum[rt] = lsum[rt] * alpha + ps;
      m2[rt] = m_new;
      // O is rescaled only when some row of the tile raised its max
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0ull) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) oacc[rt][dt][e] *= alpha;
      }
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d = 32 * dt + dgrp;
        const int cc = d >> 3, half = (d >> 2) & 1;
        const int t_lo = 16 * kb + 4 * lh + jq, t_hi = t_lo + 8;
        const dv4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (dv4s __attribute__((address_space(3))) *)(vl + t_lo * PB + ((cc ^ dswz<DH>(t_lo)) << 4) + half * 8));
        const dv4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (dv4s __attribute__((address_space(3))) *)(vl + t_hi * PB + ((cc ^ dswz<DH>(t_hi)) << 4) + half * 8));
        const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
        const V8 va = __builtin_bit_cast(V8, make_uint4(l2.x, l2.y, h2.x, h2.y));
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          if constexpr (__is_same(T, __bf16)) {
            oacc[rt][dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[rt][kb], oacc[rt][dt], 0, 0, 0);
            oacc[rt][dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pbl[rt][kb], oacc[rt][dt], 0, 0, 0);
          } else {
            oacc[rt][dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[rt][kb], oacc[rt][dt], 0, 0, 0);
            oacc[rt][dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pbl[rt][kb], oacc[rt][dt], 0, 0, 0);
          }
        }
      }
    }
  };

  // ---- pipeline: stage g in ring slot g % NSTG, loads NSTG - 1 stages ahead
#pragma unroll
  for (int i = 0; i < NSTG - 1; ++i)
    if (i < nst) {
      ensure_window(i);
      issue(i);
    }
  for (int gs = 0; gs < nst; ++gs) {
    // stage gs has landed once at most rem younger stages' loads are outstanding
    wait_stages<PER, NSTG - 2>(min(NSTG - 2, nst - 1 - gs));
    lds_barrier();  // stage gs visible to all waves; stage gs - 1 is no longer read
    const int gi = gs + NSTG - 1;
    if (gi < nst) {
      ensure_window(gi);
      issue(gi);
    }
    const unsigned char *kl = ring[gs % NSTG];
    const unsigned char *vl = kl + ST * PB;
    // the next slice's S^T chain is issued before this slice's softmax, so the matrix
    // core works while the VALU does the exp/max/sum
    Tiles st_cur = qk(kl);
#pragma unroll
    for (int b = 0; b < ST / 32; ++b) {
      Tiles st_next;
      if (b + 1 < ST / 32) st_next = qk(kl + (b + 1) * 32 * PB);
      softmax_pv(st_cur, vl + b * 32 * PB, gs * ST + 32 * b);
      st_cur = st_next;
    }
  }

#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    if (!valid[rt]) continue;
    // ---- split: the chunk's partial (unnormalised O, max, sum) for the combine kernel
    if (a.nchunk > 1) {
      const int64_t pr = ((int64_t)p * a.rows_pad + row[rt]) * a.nchunk + chunk;
      float *wo = a.ws_o + pr * DH;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f32x4 v;
          v[0] = oacc[rt][dt][4 * i]; v[1] = oacc[rt][dt][4 * i + 1];
          v[2] = oacc[rt][dt][4 * i + 2]; v[3] = oacc[rt][dt][4 * i + 3];
          *(f32x4 *)(wo + 32 * dt + 8 * i + 4 * lh) = v;
        }
      if (lh == 0) { a.ws_ml[pr * 2] = m2[rt]; a.ws_ml[pr * 2 + 1] = lsum[rt]; }
      continue;
    }
    const float inv = lsum[rt] > 0.f ? 1.0f / lsum[rt] : 0.f;
    float *op = a.out + (int64_t)l * a.o_sl + (int64_t)r * a.o_sr + (int64_t)n[rt] * a.o_sn +
                (int64_t)(h * G + g[rt]) * a.o_sh;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d0 = 32 * dt + 8 * i + 4 * lh;
        f32x4 v;
        v[0] = oacc[rt][dt][4 * i] * inv; v[1] = oacc[rt][dt][4 * i + 1] * inv;
        v[2] = oacc[rt][dt][4 * i + 2] * inv; v[3] = oacc[rt][dt][4 * i + 3] * inv;
        *(f32x4 *)(op + d0) = v;
      }
    if (lh == 0)
      a.lse[(int64_t)l * a.lse_sl + (int64_t)r * a.lse_sr + (int64_t)n[rt] * a.lse_sn + h * G + g[rt]] =
          lsum[rt] > 0.f ? (m2[rt] + __log2f(lsum[rt])) * 0.6931471805599453f : -INFINITY;
  }
}

// ------------------------------------------------------------------ split combine
// grid ceil(pairs*rows_pad/4), 256 threads: one wave per (pair, row) merging with
// attn_merge_row (DH = 0: attn_merge_row_any, the float32 path's head dims).  The decode
// kernel (a.dyn) wrote a sequence of at most one chunk's tokens itself: those rows are skipped.
template <int DH>
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
  // chunks past the sequence were never written: they hold no token of this row
  const int S_all = attn_seq_len(a, r);
  const int nc = a.dyn ? attn_dec_chunks(a, S_all) : min(a.nchunk, (S_all + a.tpc - 1) / a.tpc);
  if (a.dyn && nc <= 1) return;
  const int64_t o_off = (int64_t)l * a.o_sl + (int64_t)r * a.o_sr + (int64_t)n * a.o_sn + (int64_t)(h * a.G + g) * a.o_sh;
  const int64_t lse_off = (int64_t)l * a.lse_sl + (int64_t)r * a.lse_sr + (int64_t)n * a.lse_sn + h * a.G + g;
  if constexpr (DH == 0)
    attn_merge_row_any(a, id, nc, o_off, lse_off, lane);
  else
    attn_merge_row<DH>(a, id, nc, o_off, lse_off, lane);
}

// ------------------------------------------------------------------ generic path
// Any dtype pairing, head dims up to 512, any block size.  grid pairs * ngroups * nchunk,
// 256 threads: a workgroup takes up to NR query rows (n, g) of one (layer, request, KV
// head) pair -- a decode step's whole GQA group of up to 8 heads, so K and V are read once
// for all of its rows -- over one token chunk, 256 tokens at a time:
//   thread j: s_i = q_i . k_(t0+j) for each row i (the rows from LDS, the dot products in
//   registers as independent FMA chains), the tile's max and sum of p per row through wave
//   reductions and LDS, p_i,j into LDS; then O_i += sum_j p_i,j v_(t0+j) by token groups
//   (ceil(D/8) threads per token, 8 dims each; the groups' partial O summed in order at the
//   chunk's end).
// Online softmax in log2 units, as the matrix-core kernels; a split sequence's chunks go
// through the same workspace layout ([pair][row][chunk][D] and (max, sum)) and the combine
// launch.  Tokens in blocks the table marks invalid, and tokens a row does not see, get
// probability 0 (the V rows of invalid blocks are not read).
// NR rows per workgroup (a power of two up to AG_ROWS, the fewest that hold a pair's rows):
// the row loops are unrolled over NR, and rows past the pair's last are padding that sees
// no token.  With the row loops bounded at run time instead, the compiler walked the rows
// one at a time and re-read K and V per row; a cap of 16 rows cost a wave per SIMD (133
// registers) and measured slower than 8 on 32 and 512 rows per pair.
constexpr int AG_ROWS = 8;  // the launch switch instantiates 1, 2, 4 and 8
template <typename QT, typename KT, int NR>
__global__ void __launch_bounds__(256) attn_generic_kernel(AttnArgs a, int pairs, int ngroups) {
  extern __shared__ __attribute__((aligned(16))) float sm[];  // q rows [NR][DP], then p [NR][256]
  __shared__ float red[NR][4], redsum[NR][4];
  __shared__ int lims[NR];
  __shared__ int64_t offs[256];
  __shared__ float vred[2048];  // the token groups' partial O of one row: tp * D <= 2048
  const int D = a.D, DP = (D + 3) & ~3;
  float *qs = sm, *ps = sm + NR * DP;
  const int bid = blockIdx.x;
  const int chunk = bid % a.nchunk;
  const int grp = (bid / a.nchunk) % ngroups;
  const int p = bid / (a.nchunk * ngroups);
  if (p >= pairs) return;
  const int h = p % a.Hkv;
  const int r = (p / a.Hkv) % a.R;
  const int l = p / (a.Hkv * a.R);
  const int G = a.G;
  const int nq = attn_nq(a, r);
  const int row0 = grp * NR;
  if (row0 >= nq * G) return;
  const int nrows = min(NR, nq * G - row0);
  const int S_all = attn_seq_len(a, r);
  if (a.nchunk > 1 && chunk * a.tpc >= S_all) return;   // the combine reads only chunks with tokens
  const int c_begin = min(chunk * a.tpc, S_all);
  const int c_end = a.nchunk > 1 ? min(S_all, c_begin + a.tpc) : S_all;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  for (int i = tid; i < NR * DP; i += 256) {
    const int ri = i / DP, d = i % DP, row = row0 + ri;
    float v = 0.f;
    if (ri < nrows && d < D)
      v = (float)((const QT *)a.q)[(int64_t)l * a.q_sl + (int64_t)r * a.q_sr + (int64_t)(row / G) * a.q_sn +
                                   (int64_t)(h * G + row % G) * a.q_sh + d];
    qs[i] = v;
  }
  if (tid < NR) lims[tid] = tid < nrows ? min(attn_lim(a, r, (row0 + tid) / G, S_all), c_end) : c_begin;
  __syncthreads();
  int t_end = c_begin;  // the last token any row of the workgroup sees, plus one
  for (int i = 0; i < nrows; ++i) t_end = max(t_end, lims[i]);

  const KT *kplane = (const KT *)a.kv + (int64_t)l * a.kv_sl + (int64_t)h * a.kv_sh;
  const KT *vplane = kplane + a.kv_sv;
  const float c2 = a.scale * 1.4426950408889634f;
  // P.V mapping: tpt threads per token, each with DPT consecutive dims of its V row; tp tokens
  // in flight at a time, token j of a tile on thread group j mod tp
  constexpr int DPT = 8;
  const int tpt = (D + DPT - 1) / DPT, tp = 256 / tpt;
  const int vgrp = tid / tpt, dbase = (tid - vgrp * tpt) * DPT;
  const bool vact = vgrp < tp;
  float m2[NR], lsum[NR], acc[NR][DPT];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    m2[i] = -INFINITY;
    lsum[i] = 0.f;
#pragma unroll
    for (int e = 0; e < DPT; ++e) acc[i][e] = 0.f;
  }

  for (int t0 = c_begin; t0 < t_end; t0 += 256) {
    const int t = t0 + tid;
    int64_t off = -1;
    if (t < t_end) {
      const int ph = attn_phys(a, r, t / a.BS);
      if (ph >= 0) off = (int64_t)ph * a.kv_sb + (int64_t)(t % a.BS) * a.kv_ss;
    }
    offs[tid] = off;
    float x[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) x[i] = 0.f;
    if (off >= 0) {
      const KT *kr = kplane + off;
      int d = 0;
      // unrolled: several loads of the K row in flight per thread (bit-identical results;
      // 16 and 64 queries per pair 809 -> 549 and 907 -> 684 us, decode unchanged)
#pragma unroll 8
      for (; d + 4 <= D; d += 4) {
        const float k0 = (float)kr[d], k1 = (float)kr[d + 1], k2 = (float)kr[d + 2], k3 = (float)kr[d + 3];
#pragma unroll
        for (int i = 0; i < NR; ++i) {
          const float4 qv = *(const float4 *)&qs[i * DP + d];
          x[i] = fmaf(k0, qv.x, x[i]);
          x[i] = fmaf(k1, qv.y, x[i]);
          x[i] = fmaf(k2, qv.z, x[i]);
          x[i] = fmaf(k3, qv.w, x[i]);
        }
      }
      for (; d < D; ++d) {
        const float k0 = (float)kr[d];
#pragma unroll
        for (int i = 0; i < NR; ++i) x[i] = fmaf(k0, qs[i * DP + d], x[i]);
      }
    }
    // scaled logits (log2 units), -inf where the row does not see the token; tile max per row
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      x[i] = off >= 0 && t < lims[i] ? x[i] * c2 : -INFINITY;   // padding rows see no token
      float mx = x[i];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
      if (lane == 0) red[i][wave] = mx;
    }
    __syncthreads();
    float alpha[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const float tm = fmaxf(fmaxf(red[i][0], red[i][1]), fmaxf(red[i][2], red[i][3]));
      const float m_new = fmaxf(m2[i], tm);
      const float msafe = m_new == -INFINITY ? 0.f : m_new;
      alpha[i] = exp2f(m2[i] - msafe);
      m2[i] = m_new;
      const float pv = x[i] == -INFINITY ? 0.f : exp2f(x[i] - msafe);
      ps[i * 256 + tid] = pv;
      float sum = pv;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
      if (lane == 0) redsum[i][wave] = sum;
    }
    __syncthreads();
    // l_i += the tile's sum of p (the same four wave sums, in order, in every thread);
    // O_i[d] += sum_j p_i,j v_j[d] over the thread's tokens j = vgrp, vgrp + tp, ...
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      lsum[i] = lsum[i] * alpha[i] + ((redsum[i][0] + redsum[i][1]) + (redsum[i][2] + redsum[i][3]));
#pragma unroll
      for (int e = 0; e < DPT; ++e) acc[i][e] *= alpha[i];
    }
    const int cnt = min(256, t_end - t0);
    if (vact) {
      for (int j = vgrp; j < cnt; j += tp) {
        const int64_t oj = offs[j];
        if (oj < 0) continue;  // a token of an invalid block: p = 0 in every row
        const KT *vr = vplane + oj + dbase;
        float v[DPT];
#pragma unroll
        for (int e = 0; e < DPT; ++e) v[e] = dbase + e < D ? (float)vr[e] : 0.f;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
          const float pj = ps[i * 256 + j];
#pragma unroll
          for (int e = 0; e < DPT; ++e) acc[i][e] = fmaf(pj, v[e], acc[i][e]);
        }
      }
    }
    __syncthreads();  // ps, offs and red are rewritten by the next tile
  }

  // each row: the token groups' partial O summed in group order through LDS, then written
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    if (i >= nrows) break;  // uniform
    __syncthreads();
    if (vact) {
#pragma unroll
      for (int e = 0; e < DPT; ++e)
        if (dbase + e < D) vred[vgrp * D + dbase + e] = acc[i][e];
    }
    __syncthreads();
    const int row = row0 + i, n = row / G, g = row % G;
    if (a.nchunk > 1) {
      const int64_t pr = ((int64_t)p * a.rows_pad + row) * a.nchunk + chunk;
      float *wo = a.ws_o + pr * D;
      for (int d = tid; d < D; d += 256) {
        float o = 0.f;
        for (int gi = 0; gi < tp; ++gi) o += vred[gi * D + d];
        wo[d] = o;
      }
      if (tid == 0) { a.ws_ml[pr * 2] = m2[i]; a.ws_ml[pr * 2 + 1] = lsum[i]; }
    } else {
      float *op = a.out + (int64_t)l * a.o_sl + (int64_t)r * a.o_sr + (int64_t)n * a.o_sn + (int64_t)(h * G + g) * a.o_sh;
      const float inv = lsum[i] > 0.f ? 1.0f / lsum[i] : 0.f;
      for (int d = tid; d < D; d += 256) {
        float o = 0.f;
        for (int gi = 0; gi < tp; ++gi) o += vred[gi * D + d];
        op[d] = o * inv;
      }
      if (tid == 0)
        a.lse[(int64_t)l * a.lse_sl + (int64_t)r * a.lse_sr + (int64_t)n * a.lse_sn + h * G + g] =
            lsum[i] > 0.f ? (m2[i] + __log2f(lsum[i])) * 0.6931471805599453f : -INFINITY;
    }
  }
}

// Ring workgroup shape for a pair with rtiles 32-row tiles of query rows: waves and row
// tiles per wave.  Two tiles per wave (each K and V^T fragment read once for 64 rows)
// needs about 500 registers, one wave per SIMD, and measured 4.86 ms against 3.40 ms for
// one tile per wave at two waves per SIMD (36 layers x 32k x 128 queries): the second
// wave hides more than the halved LDS reads save.
struct RingCfg { int nw, rt; };
static RingCfg ring_cfg(int rtiles) {
  if (rtiles <= 2) return {2, 1};
  if (rtiles <= 4) return {4, 1};
  return {8, 1};
}

// Token-range split: enough (pair, row group, chunk) work items for about four rounds of
// resident workgroups (1 per CU at 8 waves, 2 at 4, 4 at 1-2 waves: the LDS stage
// buffers), chunks of at least 256 tokens, a whole number of stages each.
struct AttnSplit { int nchunk, tpc, rows_pad, ngroups; };
// compute units of the current device (256 on MI355X), queried once per device
static int device_cus() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

static AttnSplit attn_split(int pairs, int N, int G, int span, int cus) {
  AttnSplit sp;
  const int rtiles = (N * G + 31) / 32;
  if (rtiles == 1) {
    // decode kernel: DW waves per (pair, chunk), two resident workgroups per CU.  With few
    // pairs the chunks stop at about 1.5 workgroups per CU, within one round: a served decode
    // step's per-layer call (32 pairs x 4400 tokens) took 27.7 / 28.1 / 26.1 / 28.3 / 31.7 /
    // 33.7 us with 8 / 10 / 12 / 16 / 20 / 24 chunks, and 37 us with a second round (32).  With many pairs there are several rounds anyway, and at least 8 chunks per
    // pair keep the workgroups of the longest requests in a ragged batch from forming the
    // tail (a chunk holds at least one slice per wave: attn_dec_chunks).  From 16 rounds of
    // pairs on, the tail is a small part of the call and one pass per pair keeps the
    // workspace from growing with the batch (8 chunks of 256k pairs would want gigabytes).
    // The slices are interleaved over the chunks, so nothing depends on the block table's
    // width: the same sequences give the same bits however wide the table is.  Partial
    // results are kept for the N * G rows that exist.
    sp.ngroups = 1;
    sp.rows_pad = N * G;
    sp.nchunk = pairs >= 32 * cus ? 1 : std::max(8, 3 * cus / 2 / std::max(pairs, 1));
    sp.tpc = sp.nchunk > 1 ? 0 : std::max(span, 1);
    return sp;
  }
  const RingCfg cfg = ring_cfg(rtiles);
  const int tiles = cfg.nw * cfg.rt;
  const int st = tiles >= 8 ? 128 : 64;  // ring stage (RingShape<tiles>::ST)
  sp.ngroups = (rtiles + tiles - 1) / tiles;
  sp.rows_pad = sp.ngroups * tiles * 32;
  const int per_cu = tiles >= 8 ? 1 : 2;  // resident ring workgroups per CU (LDS)
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

static size_t attn_ws_bytes(int pairs, const AttnSplit &sp, int D) {
  if (sp.nchunk <= 1) return 0;
  return (size_t)pairs * sp.rows_pad * sp.nchunk * (D + 2) * sizeof(float);
}

template <typename T, typename V8, int DH>
static int launch_attn_mfma(AttnArgs a, int bs_shift, void *ws, size_t ws_bytes, hipStream_t st) {
  const int pairs = a.L * a.R * a.Hkv;
  const int rtiles = (a.N * a.G + 31) / 32;
  const bool causal = a.kv_len != nullptr;
  AttnSplit sp = attn_split(pairs, a.N, a.G, a.max_blocks * a.BS, device_cus());
  const size_t need = attn_ws_bytes(pairs, sp, DH);
  if (sp.nchunk > 1 && (!ws || ws_bytes < need)) {  // no (large enough) workspace: no split
    sp.nchunk = 1;
    sp.tpc = std::max(a.max_blocks * a.BS, 1);
  }
  a.nchunk = sp.nchunk; a.tpc = sp.tpc; a.rows_pad = sp.rows_pad;
  a.dyn = rtiles == 1 && sp.nchunk > 1;
  a.ws_o = sp.nchunk > 1 ? (float *)ws : nullptr;
  a.ws_ml = sp.nchunk > 1 ? (float *)((char *)ws + (size_t)pairs * sp.rows_pad * sp.nchunk * DH * sizeof(float)) : nullptr;
  if (rtiles == 1) {
    const int grid = pairs * sp.nchunk;
    if (causal)
      hipLaunchKernelGGL((attn_decode_kernel<T, V8, DH, true>), dim3(grid), dim3(DW * 64), 0, st, a, pairs, bs_shift);
    else
      hipLaunchKernelGGL((attn_decode_kernel<T, V8, DH, false>), dim3(grid), dim3(DW * 64), 0, st, a, pairs, bs_shift);
  } else {
#define ACTKV_ATTN(NWV, RTV)                                                                       \
  do {                                                                                             \
    const int grid = ((pairs + 7) / 8) * 8 * sp.ngroups * sp.nchunk;                               \
    if (causal)                                                                                    \
      hipLaunchKernelGGL((attn_ring_kernel<T, V8, DH, NWV, RTV, true>), dim3(grid), dim3(NWV * 64), \
                         0, st, a, pairs, sp.ngroups, bs_shift);                                   \
    else                                                                                           \
      hipLaunchKernelGGL((attn_ring_kernel<T, V8, DH, NWV, RTV, false>), dim3(grid), dim3(NWV * 64),\
                         0, st, a, pairs, sp.ngroups, bs_shift);                                   \
  } while (0)
  const RingCfg cfg = ring_cfg(rtiles);
  if (cfg.nw == 2) ACTKV_ATTN(2, 1);
  else if (cfg.nw == 4) ACTKV_ATTN(4, 1);
  else ACTKV_ATTN(8, 1);
#undef ACTKV_ATTN
  }
  int rc = actkv_check_launch();
  if (rc || sp.nchunk <= 1) return rc;
  const int64_t waves = (int64_t)pairs * sp.rows_pad;
  hipLaunchKernelGGL(attn_combine_kernel<DH>, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, a, pairs);
  return actkv_check_launch();
}

// Token split of the float32 path: about four workgroups per CU over the (pair, row group)
// items, chunks of a whole number of 256-token tiles.
// rows per workgroup of the float32 path: the fewest (a power of two, at most AG_ROWS) that
// hold a pair's N * G rows
static int attn_generic_rows(int N, int G) {
  const int64_t rows = (int64_t)N * G;
  int nr = 1;
  while (nr < AG_ROWS && nr < rows) nr *= 2;
  return nr;
}

static AttnSplit attn_split_generic(int pairs, int N, int G, int span, int cus) {
  AttnSplit sp;
  const int nr = attn_generic_rows(N, G);
  sp.ngroups = (int)(((int64_t)N * G + nr - 1) / nr);
  sp.rows_pad = sp.ngroups * nr;
  const int64_t items = (int64_t)pairs * sp.ngroups;
  const int64_t want = 4LL * cus;
  int nchunk = (int)std::min<int64_t>(std::max<int64_t>(1, (want + items - 1) / items), std::max(1, span / 256));
  int tpc = ((span + nchunk - 1) / nchunk + 255) / 256 * 256;
  tpc = std::max(tpc, 256);
  sp.nchunk = (span + tpc - 1) / tpc;
  sp.tpc = tpc;
  if (sp.nchunk <= 1) { sp.nchunk = 1; sp.tpc = std::max(span, 1); }
  return sp;
}

template <typename QT, typename KT>
static int launch_attn_generic(AttnArgs a, void *ws, size_t ws_bytes, hipStream_t st) {
  const int64_t pairs64 = (int64_t)a.L * a.R * a.Hkv;
  const int nr = attn_generic_rows(a.N, a.G);
  const int64_t groups = ((int64_t)a.N * a.G + nr - 1) / nr;
  if (pairs64 * groups > 0x7fffffffLL) return ACTKV_ERR_UNSUPPORTED;
  const int pairs = (int)pairs64;
  AttnSplit sp = attn_split_generic(pairs, a.N, a.G, a.max_blocks * a.BS, device_cus());
  const size_t need = attn_ws_bytes(pairs, sp, a.D);
  if (sp.nchunk > 1 && (!ws || ws_bytes < need || (int64_t)pairs * sp.ngroups * sp.nchunk > 0x7fffffffLL)) {
    sp.nchunk = 1;
    sp.tpc = std::max(a.max_blocks * a.BS, 1);
  }
  a.nchunk = sp.nchunk; a.tpc = sp.tpc; a.rows_pad = sp.rows_pad; a.dyn = 0;
  a.ws_o = sp.nchunk > 1 ? (float *)ws : nullptr;
  a.ws_ml = sp.nchunk > 1 ? (float *)((char *)ws + (size_t)pairs * sp.rows_pad * sp.nchunk * a.D * sizeof(float)) : nullptr;
  const size_t shm = (size_t)nr * (((a.D + 3) & ~3) + 256) * sizeof(float);
  const dim3 grid((unsigned)((int64_t)pairs * sp.ngroups * sp.nchunk));
#define ACTKV_AG(NRV) hipLaunchKernelGGL((attn_generic_kernel<QT, KT, NRV>), grid, dim3(256), shm, st, a, pairs, sp.ngroups)
  switch (nr) {
    case 1: ACTKV_AG(1); break;
    case 2: ACTKV_AG(2); break;
    case 4: ACTKV_AG(4); break;
    default: ACTKV_AG(8); break;   // AG_ROWS
  }
#undef ACTKV_AG
  int rc = actkv_check_launch();
  if (rc || sp.nchunk <= 1) return rc;
  const int64_t waves = (int64_t)pairs * sp.rows_pad;
  hipLaunchKernelGGL(attn_combine_kernel<0>, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, a, pairs);
  return actkv_check_launch();
}

template <typename QT>
static int dispatch_attn_generic(const AttnArgs &a, int kv_dtype, void *ws, size_t wb, hipStream_t st) {
  switch (kv_dtype) {
    case ACTKV_F32: return launch_attn_generic<QT, float>(a, ws, wb, st);
    case ACTKV_F16: return launch_attn_generic<QT, _Float16>(a, ws, wb, st);
    case ACTKV_BF16: return launch_attn_generic<QT, __bf16>(a, ws, wb, st);
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
  a.nchunk = 1; a.tpc = max_blocks * block_size; a.rows_pad = 0; a.dyn = 0;
  a.ws_o = nullptr; a.ws_ml = nullptr;
  const int G = a.G;
  int bs_shift = -1;
  for (int sh = 4; sh < 31; ++sh)
    if (block_size == (1 << sh)) bs_shift = sh;
  const bool vec_ok = attn_aligned16(q) && attn_aligned16(kv) && attn_aligned16(out) &&
                      q_sl % 8 == 0 && q_sr % 8 == 0 && q_sn % 8 == 0 && q_sh % 8 == 0 &&
                      kv_sl % 8 == 0 && kv_sv % 8 == 0 && kv_sb % 8 == 0 && kv_ss % 8 == 0 &&
                      kv_sh % 8 == 0 && o_sl % 4 == 0 && o_sr % 4 == 0 && o_sn % 4 == 0 && o_sh % 4 == 0;
  const bool mfma_ok = q_dtype == kv_dtype && (kv_dtype == ACTKV_BF16 || kv_dtype == ACTKV_F16) &&
                       (D == 128 || D == 64) && G >= 1 && vec_ok && bs_shift >= 0;
  if (mfma_ok) {
    void *ws = workspace;
    const size_t wb = workspace_bytes;
    if (kv_dtype == ACTKV_BF16)
      return D == 64 ? launch_attn_mfma<__bf16, bf16x8, 64>(a, bs_shift, ws, wb, st)
                     : launch_attn_mfma<__bf16, bf16x8, 128>(a, bs_shift, ws, wb, st);
    return D == 64 ? launch_attn_mfma<_Float16, f16x8, 64>(a, bs_shift, ws, wb, st)
                   : launch_attn_mfma<_Float16, f16x8, 128>(a, bs_shift, ws, wb, st);
  }
  switch (q_dtype) {
    case ACTKV_F32: return dispatch_attn_generic<float>(a, kv_dtype, workspace, workspace_bytes, st);
    case ACTKV_F16: return dispatch_attn_generic<_Float16>(a, kv_dtype, workspace, workspace_bytes, st);
    default: return dispatch_attn_generic<__bf16>(a, kv_dtype, workspace, workspace_bytes, st);
  }
}

extern "C" size_t actkv_paged_attention_workspace_size(int L, int R, int N, int Hq, int Hkv, int D,
                                                       int max_blocks, int block_size) {
  if (L < 1 || R < 1 || N < 1 || Hkv < 1 || Hq % Hkv != 0 || max_blocks < 1 || block_size < 1) return 0;
  const int G = Hq / Hkv;
  if (G < 1 || D > 512) return 0;
  if ((int64_t)max_blocks * block_size > 0x7fffffffLL) return 0;
  const int pairs = L * R * Hkv;
  // head dims 128 and 64: the matrix-core split; others: the float32 path's split
  if (D == 128 || D == 64)
    return attn_ws_bytes(pairs, attn_split(pairs, N, G, max_blocks * block_size, device_cus()), D);
  return attn_ws_bytes(pairs, attn_split_generic(pairs, N, G, max_blocks * block_size, device_cus()), D);
}
