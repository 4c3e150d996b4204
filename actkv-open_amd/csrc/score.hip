// LSE-recovery scoring on a paged KV cache (ActKV Algorithm 3) for gfx950.
//
// Reference: actkv/kernels/lse_attn.py:85-163.  The reference launches one
// Triton program per (request, logical block, KV head) and folds ONE action
// query per launch, so K is re-read from HBM once per action token.  Here one
// workgroup owns a (layer, request, KV head) pair -- or, for small tiles, several
// KV heads of one (layer, request) -- and a token range, holds the whole
// action-query tile (N queries x G group heads per head) on chip and reads the
// range's K rows from HBM exactly once.  Two MFMA kernels: above 384 query rows,
// and up to 128, the tile sits in registers while K chunks are shared through LDS
// (score_qreg_kernel: fewer LDS reads per MFMA; the matrix cores bound it above
// 384 rows, HBM up to 128); from 129 to 384 rows each wave streams its own K
// slices into registers against the tile in LDS (score_kslice_kernel).  Both compute
//
//   acc[row, t] = q_row . k_t - lse_row / scale            (bf16/fp16 MFMA, fp32 acc)
//   p[n, t]     = exp2(scale*log2(e) * max_g acc[(n,g), t]) (max over the GQA group
//                                                           before the exp: exp is monotonic)
//   sum[t]      = sum_n p[n, t]                              (per-wave sums + LDS)
//   out[t]      = (out[t] * n_seen + sum[t]) / (n_seen + nq) (== nq reference folds)
//
// Groups of 8 and 16 heads run on the query-register kernel only: a query's rows
// span both halves of a wave, and their max is taken across the halves.  Groups of
// 3, 5-7 and 9-15 take that kernel too, laid out as 4, 8 and 16 rows per query
// (padding rows load no query and start at -inf).  The generic kernels cover every
// other shape/dtype (fp32 caches or queries, head dims other than 64 and 128, groups
// above 16, blocks that are not a power of two from 16 up) in float32 and follow the
// reference fold order exactly: for each query in turn,
// out += (p - out) / (n_seen + n + 1).  score_generic_rows_kernel (head dims that are a
// multiple of 4 up to 512) keeps a chunk of query rows' dot products in registers;
// score_generic_kernel takes the rest one query at a time.
#include "common.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace actkv {

// Longest token range of one MFMA workgroup (its block-table slice holds
// MFMA_MAX_TOKENS / 16 entries, one per thread of the 512).
constexpr int MFMA_MAX_TOKENS = 8192;

struct ScoreArgs {
  const void *q;
  int64_t q_sl, q_sr, q_sn, q_sh;
  const void *kv;
  int64_t kv_sl, kv_sb, kv_ss, kv_sh;
  int64_t num_blocks;
  const int32_t *bt;
  int64_t bt_sr;
  int max_blocks;
  const int32_t *seq_used;
  const float *lse;
  int64_t lse_sl, lse_sr, lse_sn;
  float *out;
  int64_t out_sl, out_sr, out_sh;
  const int32_t *n_seen;
  const int32_t *n_valid;
  const int32_t *kv_len;
  int L, R, N, Hq, Hkv, D, G, BS;
  float scale;
  int qc0, qcn;  // query chunk [qc0, qc0+qcn) handled by this launch (MFMA path)
};

// IEEE maximum (NaN-propagating, as torch's amax): lowers to v_maximum3_f32 on
// gfx950 without the operand canonicalisation fmaxf needs.
__device__ __forceinline__ float vmax(float x, float y) { return __builtin_elementwise_maximum(x, y); }

// Workgroup barrier for LDS hand-overs that leaves VM loads in flight: this wave's LDS
// reads and writes complete (lgkmcnt(0)) and at most VM of its vector memory operations
// are outstanding, then s_barrier; the empty asm statements keep the compiler from moving
// memory accesses across it.  __syncthreads() would fence every address space, and its
// fence waits vmcnt(0) (loads into LDS write LDS too), draining every K chunk in flight.
// Loads from global memory into LDS (lane i writes bytes [i*W, i*W + W) at lds_addr,
// W = 16 or 4).  Issued as assembly so the compiler's wait insertion does not track them:
// it cannot tell which LDS array such a load writes, and waits for all of them (vmcnt(0))
// before any later LDS access.  Every wait for these loads is explicit in the kernel.
// M0 carries the LDS address; the compiler reserves M0 (a clobber of it is not honoured),
// so the statement saves and restores it.
__device__ __forceinline__ void load_lds16(const void *gptr, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved) : "v"(gptr), "s"(lds_addr) : "memory");
}
__device__ __forceinline__ void load_lds4(const void *gptr, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved) : "v"(gptr), "s"(lds_addr) : "memory");
}
__device__ __forceinline__ uint32_t lds_address(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

template <int VM>
__device__ __forceinline__ void lds_barrier() {
  static_assert(VM >= 0 && VM < 16, "vmcnt low bits");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0070 | VM);   // vmcnt(VM) expcnt(7) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ int seq_len_of(const ScoreArgs &a, int r) {
  int s = a.seq_used[r];
  int span = a.max_blocks * a.BS;
  return s < 0 ? 0 : (s > span ? span : s);
}

// ------------------------------------------------------------------ generic
// grid (ceil(span/256), L*R*Hkv), 256 threads; one thread per token slot.
template <typename QT, typename KT>
__global__ void __launch_bounds__(256) score_generic_kernel(ScoreArgs a) {
  extern __shared__ float qs[];  // [G*D] current query rows (fp32) then [G] lse
  const int pair = blockIdx.y;
  const int h = pair % a.Hkv;
  const int r = (pair / a.Hkv) % a.R;
  const int l = pair / (a.Hkv * a.R);
  const int S = seq_len_of(a, r);
  if ((int64_t)blockIdx.x * 256 >= S) return;
  const int nq_all = a.n_valid ? min(max(a.n_valid[r], 0), a.N) : a.N;
  if (nq_all == 0) return;
  const int t = blockIdx.x * 256 + threadIdx.x;
  const int G = a.G, D = a.D;
  float *lse_s = qs + G * D;

  bool valid = t < S;
  const KT *krow = nullptr;
  if (valid) {
    const int64_t phys = a.bt[(int64_t)r * a.bt_sr + t / a.BS];
    if (phys < 0 || phys >= a.num_blocks) {
      valid = false;
    } else {
      krow = (const KT *)a.kv + (int64_t)l * a.kv_sl + phys * a.kv_sb +
             (int64_t)(t % a.BS) * a.kv_ss + (int64_t)h * a.kv_sh;
    }
  }
  float *optr = a.out + (int64_t)l * a.out_sl + (int64_t)r * a.out_sr + (int64_t)h * a.out_sh + t;
  float acc = valid ? *optr : 0.f;
  const int n0 = a.n_seen[r];
  const QT *qbase = (const QT *)a.q + (int64_t)l * a.q_sl + (int64_t)r * a.q_sr;
  const float *lbase = a.lse + (int64_t)l * a.lse_sl + (int64_t)r * a.lse_sr;

  for (int n = 0; n < nq_all; ++n) {
    __syncthreads();
    for (int i = threadIdx.x; i < G * D; i += 256) {
      const int g = i / D, d = i % D;
      qs[i] = (float)qbase[(int64_t)n * a.q_sn + (int64_t)(h * G + g) * a.q_sh + d];
    }
    if (threadIdx.x < G) lse_s[threadIdx.x] = lbase[(int64_t)n * a.lse_sn + h * G + threadIdx.x];
    __syncthreads();
    if (valid) {
      float p = 0.f;
      if (!a.kv_len || t < a.kv_len[(int64_t)r * a.N + n]) {
        for (int g = 0; g < G; ++g) {
          float dot = 0.f;
          for (int d = 0; d < D; ++d) dot = fmaf((float)krow[d], qs[g * D + d], dot);
          p = fmaxf(p, expf(dot * a.scale - lse_s[g]));
        }
      }
      acc = acc + (p - acc) / (float)(n0 + n + 1);
    }
  }
  if (valid) *optr = acc;
}

// ------------------------------------------------------------------ generic, query rows in chunks
// The same computation and fold order as score_generic_kernel, for head dims that are a
// multiple of 4 up to 512: grid (ceil(span/256), L*R*Hkv), 256 threads, one thread per
// token slot.  The query rows (n, g) go through LDS ROWS at a time (a power of two; qc
// whole queries of gc group heads each: gc = min(G, ROWS), qc = ROWS / gc; a group wider
// than ROWS takes one query per chunk and several chunks of heads, the running max carried
// between them).  A thread walks its K row once per chunk, four dims per step, and keeps the
// chunk's ROWS dot products in registers: K is read once per ROWS rows instead of once
// per row, and the dot products are independent FMA chains.  With a float32 cache or
// queries each dot product still sums its dims in order, so the scores equal
// score_generic_kernel's.  When q and K share a 16-bit dtype the query rows sit in LDS as
// dim pairs and the products are packed two-element dots (v_dot2c_f32_bf16 / _f16:
// a.x * b.x + a.y * b.y + c in float32), within 1e-6 relative of the in-order sums.
__device__ __forceinline__ float dot2_acc(uint32_t k, uint32_t q, float c, __bf16) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, k), __builtin_bit_cast(bf2, q), c, false);
}
__device__ __forceinline__ float dot2_acc(uint32_t k, uint32_t q, float c, _Float16) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, k), __builtin_bit_cast(h2, q), c, false);
}

template <typename QT, typename KT, int ROWS>
__global__ void __launch_bounds__(256) score_generic_rows_kernel(ScoreArgs a, int gc) {
  // [ROWS][D] fp32 query rows (packed: [ROWS][D/2] dim pairs), then [ROWS] lse, [ROWS] kv_len
  extern __shared__ __attribute__((aligned(16))) float qrows[];
  constexpr bool PACK = __is_same(QT, KT) && (__is_same(KT, __bf16) || __is_same(KT, _Float16));
  const int pair = blockIdx.y;
  const int h = pair % a.Hkv;
  const int r = (pair / a.Hkv) % a.R;
  const int l = pair / (a.Hkv * a.R);
  const int S = seq_len_of(a, r);
  if ((int64_t)blockIdx.x * 256 >= S) return;
  const int nq_all = a.n_valid ? min(max(a.n_valid[r], 0), a.N) : a.N;
  if (nq_all == 0) return;
  const int t = blockIdx.x * 256 + threadIdx.x;
  const int G = a.G, D = a.D;
  const int qc = ROWS / gc;
  float *lse_s = qrows + ROWS * D;
  int *kvl_s = (int *)(lse_s + ROWS);

  bool valid = t < S;
  const KT *krow = nullptr;
  if (valid) {
    const int64_t phys = a.bt[(int64_t)r * a.bt_sr + t / a.BS];
    if (phys < 0 || phys >= a.num_blocks) {
      valid = false;
    } else {
      krow = (const KT *)a.kv + (int64_t)l * a.kv_sl + phys * a.kv_sb +
             (int64_t)(t % a.BS) * a.kv_ss + (int64_t)h * a.kv_sh;
    }
  }
  float *optr = a.out + (int64_t)l * a.out_sl + (int64_t)r * a.out_sr + (int64_t)h * a.out_sh + t;
  float acc = valid ? *optr : 0.f;
  const int n0 = a.n_seen[r];
  const QT *qbase = (const QT *)a.q + (int64_t)l * a.q_sl + (int64_t)r * a.q_sr;
  const float *lbase = a.lse + (int64_t)l * a.lse_sl + (int64_t)r * a.lse_sr;

  float carry = -INFINITY;  // max over the earlier head chunks of a group wider than ROWS
  for (int nc = 0; nc < nq_all; nc += qc) {
    const int qn = min(qc, nq_all - nc);
    for (int g0 = 0; g0 < G; g0 += gc) {
      const int gn = min(gc, G - g0);
      const bool last = g0 + gc >= G;
      __syncthreads();
      if constexpr (PACK) {
        uint32_t *qp = (uint32_t *)qrows;
        const int D2 = D / 2;
        for (int i = threadIdx.x; i < ROWS * D2; i += 256) {
          const int row = i / D2, d = 2 * (i % D2), j = row / gc, g = row % gc;
          uint32_t v = 0;
          if (j < qn && g < gn) {
            const QT *src = qbase + (int64_t)(nc + j) * a.q_sn + (int64_t)(h * G + g0 + g) * a.q_sh + d;
            v = (uint32_t)__builtin_bit_cast(uint16_t, src[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, src[1]) << 16);
          }
          qp[i] = v;
        }
      } else {
        for (int i = threadIdx.x; i < ROWS * D; i += 256) {
          const int row = i / D, d = i % D, j = row / gc, g = row % gc;
          qrows[i] = j < qn && g < gn
                         ? (float)qbase[(int64_t)(nc + j) * a.q_sn + (int64_t)(h * G + g0 + g) * a.q_sh + d]
                         : 0.f;
        }
      }
      if (threadIdx.x < ROWS) {
        const int row = threadIdx.x, j = row / gc, g = row % gc;
        lse_s[row] = j < qn && g < gn ? lbase[(int64_t)(nc + j) * a.lse_sn + h * G + g0 + g] : 0.f;
        kvl_s[row] = row < qn && a.kv_len ? a.kv_len[(int64_t)r * a.N + nc + row] : 0x7fffffff;  // query row's limit
      }
      __syncthreads();
      if (!valid) continue;
      float dot[ROWS];
#pragma unroll
      for (int i = 0; i < ROWS; ++i) dot[i] = 0.f;
      // up to 32 rows the dim loop is unrolled by 8, so that several loads of the K row are in
      // flight (one query of a small group: 157 -> 33 us per head-dim-256 32k layer); at 64 rows
      // unrolling takes more than 256 registers and measured slower
      constexpr int UNR = ROWS <= 32 ? 8 : 1;
      if constexpr (PACK) {
        const uint32_t *qp = (const uint32_t *)qrows;
        const int D2 = D / 2;
#pragma unroll UNR
        for (int d = 0; d < D; d += 4) {
          const uint32_t k01 = (uint32_t)__builtin_bit_cast(uint16_t, krow[d]) |
                               ((uint32_t)__builtin_bit_cast(uint16_t, krow[d + 1]) << 16);
          const uint32_t k23 = (uint32_t)__builtin_bit_cast(uint16_t, krow[d + 2]) |
                               ((uint32_t)__builtin_bit_cast(uint16_t, krow[d + 3]) << 16);
#pragma unroll
          for (int i = 0; i < ROWS; ++i) {
            const uint2 qv = *(const uint2 *)&qp[i * D2 + d / 2];
            dot[i] = dot2_acc(k01, qv.x, dot[i], KT{});
            dot[i] = dot2_acc(k23, qv.y, dot[i], KT{});
          }
        }
      } else {
#pragma unroll UNR
        for (int d = 0; d < D; d += 4) {
          const float k0 = (float)krow[d], k1 = (float)krow[d + 1], k2 = (float)krow[d + 2], k3 = (float)krow[d + 3];
#pragma unroll
          for (int i = 0; i < ROWS; ++i) {
            const float4 qv = *(const float4 *)&qrows[i * D + d];
            dot[i] = fmaf(k0, qv.x, dot[i]);
            dot[i] = fmaf(k1, qv.y, dot[i]);
            dot[i] = fmaf(k2, qv.z, dot[i]);
            dot[i] = fmaf(k3, qv.w, dot[i]);
          }
        }
      }
      // rows in (query, head) order: the group max, then each whole query folds in turn
      float cur = carry;
      int k = 0, j = 0;
#pragma unroll
      for (int i = 0; i < ROWS; ++i) {
        if (k < gn) cur = vmax(cur, dot[i] * a.scale - lse_s[i]);
        if (++k == gc) {
          if (j < qn) {
            if (last) {
              const float p = t < kvl_s[j] ? expf(cur) : 0.f;
              acc = acc + (p - acc) / (float)(n0 + nc + j + 1);
              carry = -INFINITY;
            } else {
              carry = cur;
            }
          }
          k = 0;
          cur = -INFINITY;
          ++j;
        }
      }
    }
  }
  if (valid) *optr = acc;
}

// ------------------------------------------------------------------ MFMA, K slices in registers
// For query tiles of at most 384 rows.  One workgroup (NW waves) owns a (layer, request, KV head) pair and a
// token range.  The pair's whole action-query tile -- rows (query n, group head g),
// nq*G <= ROWS of them, head_dim 128, bf16/fp16 -- is staged ONCE into LDS
// (rows padded to 272 bytes: conflict-free A-operand reads), with the
// accumulator seeds -lse/scale (-inf for padding rows, which then add
// exp2(-inf) = 0) and the pair's slice of the block table.  After that single
// barrier each wave works alone on 32*TT-token slices of the range: it loads the
// slice's K rows straight from HBM into MFMA B-operand registers (double
// buffered: the next slice is in flight while this one is multiplied), sweeps all
// 32-row tiles of the query tile from LDS with v_mfma_f32_32x32x16 (the shape
// that reaches the bf16 peak on gfx950), and writes the slice's running means.
//
// v_mfma_f32_32x32x16 lane layout: lane L supplies A[L%32][8*(L/32)+j] and
// B[8*(L/32)+j][L%32] (j < 8) and receives D[8*(r/4) + 4*(L/32) + r%4][L%32] in
// register r < 16.  Rows are ordered (n, g); with G = 4 each aligned group of
// four rows is one query's four group heads, so a lane holds four queries x
// four heads at one token: the GQA max is in-register and
// max_g exp(x_g) = exp(max_g x_g) costs one exp per (query, token).
template <typename T, typename V8, int G, int ROWS, bool CAUSAL, int NW, int TT>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW / 4, NW / 4)))
score_kslice_kernel(ScoreArgs a, int tpw, int cpp, int pairs, int bs_shift) {
  // NW waves (NW/4 per SIMD), TT 32-token tiles per wave slice
  constexpr int SLICE = TT * 32, KS = 8, MAXBT = MFMA_MAX_TOKENS / 16 + 2;
  constexpr int QG = 4 / G;  // queries in an aligned group of four rows
  // query rows are padded to 272 bytes: 16 consecutive rows then start in 16
  // distinct 16-byte bank groups (conflict-free A reads) and every A-operand
  // read of a tile is a constant offset from one per-lane base address
  constexpr int QROW = 272;
  __shared__ __attribute__((aligned(16))) unsigned char qs[ROWS * QROW];
  __shared__ __attribute__((aligned(16))) float cs[ROWS];
  __shared__ __attribute__((aligned(16))) int ls[CAUSAL ? ROWS : 4];
  __shared__ int bts[MAXBT];

  // XCD-aware work mapping: all token ranges of one (layer, request, head)
  // pair land on the same XCD (blockIdx % 8), so its query tile is fetched
  // from HBM into that XCD's L2 once.
  const int bid = blockIdx.x;
  const int xcd = bid & 7, jj = bid >> 3;
  const int p = (jj / cpp) * 8 + xcd;
  const int chunk = jj % cpp;
  if (p >= pairs) return;
  const int h = p % a.Hkv;
  const int r = (p / a.Hkv) % a.R;
  const int l = p / (a.Hkv * a.R);
  const int S = seq_len_of(a, r);
  const int t_begin = chunk * tpw;
  if (t_begin >= S) return;
  const int t_end = min(t_begin + tpw, S);
  const int nq_all = a.n_valid ? min(max(a.n_valid[r], 0), a.N) : a.N;
  const int nq = min(max(nq_all - a.qc0, 0), a.qcn);
  if (nq <= 0) return;
  const int n0 = a.n_seen[r] + min(nq_all, a.qc0);
  const int BS = a.BS;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lcol = lane & 31, lh = lane >> 5;
  const int rows = nq * G;
  // an even number of 32-row tiles keeps the two-tile software pipeline
  // branch-free; padding rows have zero queries and -inf seeds
  const int rtiles = (((rows + 31) >> 5) + 1) & ~1;

  // ---- stage the query tile, the accumulator seeds and the block-table slice
  {
    const T *qbase = (const T *)a.q + (int64_t)l * a.q_sl + (int64_t)r * a.q_sr;
    for (int e = tid; e < rtiles * 32 * 16; e += NW * 64) {
      const int row = e >> 4, pc = e & 15;
      const int n = row / G, g = row % G;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (n < nq)
        v = *(const uint4 *)(qbase + (int64_t)(a.qc0 + n) * a.q_sn + (int64_t)(h * G + g) * a.q_sh + pc * 8);
      *(uint4 *)(&qs[row * QROW + pc * 16]) = v;
    }
    const float *lbase = a.lse + (int64_t)l * a.lse_sl + (int64_t)r * a.lse_sr;
    const float inv_scale = 1.0f / a.scale;
    for (int row = tid; row < rtiles * 32; row += NW * 64) {
      const int n = row / G, g = row % G;
      cs[row] = n < nq ? -lbase[(int64_t)(a.qc0 + n) * a.lse_sn + h * G + g] * inv_scale : -INFINITY;
      if constexpr (CAUSAL) ls[row] = n < nq ? a.kv_len[(int64_t)r * a.N + a.qc0 + n] : 0;
    }
    const int b0 = t_begin >> bs_shift;
    const int nbt = ((t_end - 1) >> bs_shift) - b0 + 1;
    const int32_t *btr = a.bt + (int64_t)r * a.bt_sr;
    for (int i = tid; i < nbt; i += NW * 64) {
      const int64_t phys = btr[b0 + i];
      bts[i] = (phys >= 0 && phys < a.num_blocks) ? (int)phys : -1;
    }
  }
  __syncthreads();

  const T *kbase = (const T *)a.kv + (int64_t)l * a.kv_sl + (int64_t)h * a.kv_sh + lh * 8;
  const int b0 = t_begin >> bs_shift;
  const int nbt = ((t_end - 1) >> bs_shift) - b0 + 1;
  const float c2 = a.scale * 1.4426950408889634f;
  float *obase = a.out + (int64_t)l * a.out_sl + (int64_t)r * a.out_sr + (int64_t)h * a.out_sh;
  const float fn0 = (float)n0, fden = (float)(n0 + nq);

  // B operands of one slice: kf[tt][ks] = K[token s+32tt+lcol][16ks + 8lh .. +8].
  // Unconditional loads (no branch) keep the compiler's wait counts exact, so the
  // next slice stays in flight: a token past t_end, or in a block the table marks
  // invalid, reads row 0 of block 0 instead and its output column is never written.
  auto load_slice = [&](V8 (&kf)[TT][KS], int s) {
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const int tb = s + tt * 32;           // 32-token tile: whole blocks when bs >= 32,
      const int t = tb + lcol;              // else two blocks (per-lane block index)
      const int bi = min((t >> bs_shift) - b0, nbt - 1);
      int phys = bts[bi];
      const bool ok = t < t_end && phys >= 0;
      phys = ok ? phys : 0;
      const int slot = ok ? (t & (BS - 1)) : 0;
      const T *kp = kbase + (int64_t)phys * a.kv_sb + (int64_t)slot * a.kv_ss;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[tt][ks] = *(const V8 *)(kp + ks * 16);
    }
  };

  // A operands and seeds of one 32-row tile
  auto load_a = [&](int jt, V8 (&af)[KS], f32x16 &c, int (&lim)[4][QG]) {
    const unsigned char *qrow = qs + (jt * 32 + lcol) * QROW + lh * 16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) af[ks] = *(const V8 *)(qrow + ks * 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 v = *(const f32x4 *)(&cs[jt * 32 + 8 * i + 4 * lh]);
      c[4 * i + 0] = v[0]; c[4 * i + 1] = v[1]; c[4 * i + 2] = v[2]; c[4 * i + 3] = v[3];
      if constexpr (CAUSAL) {
#pragma unroll
        for (int qg = 0; qg < QG; ++qg) lim[i][qg] = ls[jt * 32 + 8 * i + 4 * lh + qg * G];
      }
    }
  };
  auto mfma_tile = [&](const V8 (&kf)[TT][KS], const V8 (&af)[KS], const f32x16 &c, f32x16 (&acc)[TT]) {
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) acc[tt] = c;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        if constexpr (__is_same(T, __bf16))
          acc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks], kf[tt][ks], acc[tt], 0, 0, 0);
        else
          acc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[ks], kf[tt][ks], acc[tt], 0, 0, 0);
      }
    }
  };
  auto post = [&](const f32x16 (&acc)[TT], const int (&lim)[4][QG], int s, float (&psum)[TT]) {
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const int t = s + tt * 32 + lcol;
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a0 = acc[tt][4 * i], a1 = acc[tt][4 * i + 1], a2 = acc[tt][4 * i + 2], a3 = acc[tt][4 * i + 3];
        if constexpr (G == 4) {
          const float e = __builtin_amdgcn_exp2f(vmax(vmax(a0, a1), vmax(a2, a3)) * c2);
          if constexpr (CAUSAL) sum += t < lim[i][0] ? e : 0.f;
          else sum += e;
        } else if constexpr (G == 2) {
          const float e0 = __builtin_amdgcn_exp2f(vmax(a0, a1) * c2);
          const float e1 = __builtin_amdgcn_exp2f(vmax(a2, a3) * c2);
          if constexpr (CAUSAL) sum += (t < lim[i][0] ? e0 : 0.f) + (t < lim[i][1] ? e1 : 0.f);
          else sum += e0 + e1;
        } else {
          const float v[4] = {a0, a1, a2, a3};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float e = __builtin_amdgcn_exp2f(v[j] * c2);
            if constexpr (CAUSAL) sum += t < lim[i][j] ? e : 0.f;
            else sum += e;
          }
        }
      }
      psum[tt] += sum;
    }
  };
  // One pipeline block: the 8*TT MFMAs of row tile j, the exp/max/sum of tile
  // j-1 and the 12 LDS reads of tile j+1, interleaved so the VALU work and the
  // LDS traffic co-issue with the matrix core.
  auto schedule_block = [&]() {
    if constexpr (TT == 1) {  // 8 MFMAs, 12 DS reads, ~30 VALU
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    } else {                  // 16 MFMAs, 12 DS reads, ~60 VALU
#pragma unroll
      for (int i = 0; i < 12; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      }
    }
  };

  auto process_slice = [&](const V8 (&kf)[TT][KS], int s) {
    // the running-mean update reads the slice's old scores: fetch them now (clamped
    // in-bounds address, unconditional) so the read is long done when they are used
    const int t_own = s + (TT == 2 ? lh * 32 : 0) + lcol;
    const float old = obase[min(t_own, t_end - 1)];
    float psum[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) psum[tt] = 0.f;
    V8 afA[KS], afB[KS];
    f32x16 cA, cB, accA[TT], accB[TT];
    int limA[4][QG], limB[4][QG];
    // rtiles is even: tile 0 (prologue), pairs (1,2) .. (rt-3, rt-2), tile rt-1
    // (epilogue); even tiles use the A buffers, odd tiles the B buffers
    load_a(0, afA, cA, limA);
    load_a(1, afB, cB, limB);
    mfma_tile(kf, afA, cA, accA);
    for (int jt = 1; jt + 1 < rtiles; jt += 2) {
      mfma_tile(kf, afB, cB, accB);
      post(accA, limA, s, psum);
      load_a(jt + 1, afA, cA, limA);
      schedule_block();
      mfma_tile(kf, afA, cA, accA);
      post(accB, limB, s, psum);
      load_a(jt + 2, afB, cB, limB);
      schedule_block();
    }
    mfma_tile(kf, afB, cB, accB);
    post(accA, limA, s, psum);
    post(accB, limB, s, psum);
    // sum the two lane halves (the queries) of each token; with TT = 2 half lh owns
    // token tile lh of the slice, with TT = 1 the first half writes
    float mine = 0.f;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const float v = psum[tt] + __shfl_xor(psum[tt], 32, 64);
      mine = (TT == 1 || lh == tt) ? v : mine;
    }
    // a token in a block the table marks invalid keeps its score, as in the other kernels
    if (t_own < t_end && (TT == 2 || lh == 0) && bts[(t_own >> bs_shift) - b0] >= 0)
      obase[t_own] = (old * fn0 + mine) / fden;
  };

  const int step = NW * SLICE;
  int s = t_begin + wave * SLICE;
  if (s >= t_end) return;
  V8 ka[TT][KS], kb[TT][KS];
  load_slice(ka, s);
  for (;;) {
    load_slice(kb, s + step);   // past the end it reads harmless in-bounds rows
    process_slice(ka, s);
    s += step;
    if (s >= t_end) break;
    load_slice(ka, s + step);
    process_slice(kb, s);
    s += step;
    if (s >= t_end) break;
  }
}

// ------------------------------------------------------------------ MFMA, query tile in registers
// One workgroup of 8 waves (2 per SIMD) owns HP KV heads of one (layer, request) and a
// token range.  Each head's action-query tile -- rows (query n, group head g), nq*G of
// them, head_dim 128, bf16/fp16 -- is split into row groups of 64 rows; the workgroup
// holds RG row groups (RG/HP per head) and splits its 8 waves over RG row groups x 8/RG
// token groups: wave (rg, tg) keeps row group rg's two 32-row tiles as MFMA A operands in
// registers for the whole range, with their accumulator seeds -lse/scale (-inf for
// padding rows, which then add exp2(-inf) = 0) as the C operand of each chain's first
// MFMA, and multiplies the 32-token tiles tg, tg + 8/RG, ... of every chunk of its head.
// With HP = 1: RG = 8 for 385..512 rows, 4 up to 256 and 2 up to 128.  With HP = 2 or 4
// (up to 256 or 128 rows) every wave still holds 64 rows and multiplies every tile of
// a chunk, and each token's K is read as HP heads' contiguous 256-byte pieces.
//
// K streams through LDS in chunks of CH tokens, NBUF - 1 chunks in flight: the waves
// load chunk c+NBUF-1 straight from HBM into LDS (global_load_lds_dwordx4) while they
// multiply chunk c, and one barrier per chunk hands a chunk over.  Two layouts: 1 KiB B
// fragments, [tile][k step][lane] x 16 bytes (HP = 1 only), so every fragment read
// (ds_read_b128) is one contiguous 1 KiB; or whole token rows of HP x 256 bytes with
// each head's 16-byte columns XOR-swizzled by token.  Both are conflict-free, and every
// fragment read feeds two MFMAs (one per row tile).
//
// v_mfma_f32_32x32x16 lane layout: lane L supplies A[L%32][8*(L/32)+j] and
// B[8*(L/32)+j][L%32] (j < 8) and receives D[8*(r/4) + 4*(L/32) + r%4][L%32] in
// register r < 16.  Rows are ordered (n, g); with G = 4 each aligned group of
// four rows is one query's four group heads, so a lane holds four queries x four
// heads at one token: the GQA max is in-register and max_g exp(x_g) =
// exp(max_g x_g) costs one exp per (query, token).
//
// Per 32-token tile a wave runs the MFMA chain of row tile 0 beside the
// exp/max/sum of row tile 1 of the previous tile, then the chain of row tile 1
// beside the exp/max/sum of row tile 0 and the B-fragment reads of the next
// tile.  Per-token partial sums (one per row group and lane half) go to LDS at
// the end of the chunk; after the next barrier the first HP x CH threads add each
// head's in a fixed order and write the running means.
template <typename T, typename V8, int G, bool CAUSAL, int RG, int NBUF, bool SWZ, int CH, int HP, int DH = 128>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
score_qreg_kernel(ScoreArgs a, int tpw, int cpp, int pairs, int bs_shift) {
  // QG: queries in an aligned group of four output rows (G <= 4); with G = 8 a query's
  // heads span two such groups, one in each half of the wave, with G = 16 four (two in
  // each half)
  constexpr int NW = 8, TG = NW / RG, KS = DH / 16, QG = G >= 4 ? 1 : 4 / G;
  static_assert(DH == 64 || DH == 128, "head dims");
  constexpr int PB = DH * 2;            // bytes of one head's piece of a token row
  constexpr int NC = PB / 16;           // its 16-byte columns
  constexpr int NCS = NC == 16 ? 4 : 3;  // log2(NC)
  static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "group sizes");
  static_assert(RG == 2 || RG == 4 || RG == 8, "row groups");
  static_assert(HP == 1 || HP == 2 || HP == 4 || HP == 8, "heads per workgroup");
  static_assert(RG % HP == 0 && (HP == 1 || SWZ), "whole row groups per head; packed heads use rows");
  static_assert(NBUF >= 2 && NBUF <= 4, "K chunk buffers");
  static_assert(CH == 32 || CH == 64 || CH == 128 || CH == 256, "tokens per chunk");
  constexpr int RGH = RG / HP;          // row groups per head
  constexpr int TPC = CH / 32;          // 32-token tiles per chunk
  constexpr int NT = TPC / TG;          // tiles per wave per chunk
  static_assert(NT >= 1 && NT * TG == TPC, "token groups");
  constexpr int HROW = HP * PB;         // bytes of one token's HP head pieces
  constexpr int CHB = CH * HROW;        // bytes of one chunk
  constexpr int LPW = CHB / 1024 / NW;  // 1 KiB loads per wave per chunk
  static_assert(LPW * 1024 * NW == CHB, "whole loads per wave");
  constexpr int NRED = 2 * RG;          // partial sums per token and head pack
  constexpr int NOLD = HP * CH / 64;    // 256-byte loads of the old means per chunk
  static_assert(NOLD * 64 == HP * CH, "whole old-mean loads");
  static_assert(SWZ || KS % LPW == 0, "a wave's fragment loads stay within one tile");
  // the K buffers are distinct arrays: the compiler then knows that reads of one
  // need not wait for the loads in flight into the others
  __shared__ __attribute__((aligned(16))) unsigned char kbuf_a[CHB];
  __shared__ __attribute__((aligned(16))) unsigned char kbuf_b[CHB];
  __shared__ __attribute__((aligned(16))) unsigned char kbuf_c[NBUF >= 3 ? CHB : 16];
  __shared__ __attribute__((aligned(16))) unsigned char kbuf_d[NBUF >= 4 ? CHB : 16];
  __shared__ float red[2][NRED][CH];
  __shared__ float oldm[8][HP * CH];   // running means of the chunks in flight, [head][token]; ring of 8 >= NBUF + 1
  __shared__ int bts[MFMA_MAX_TOKENS / 16];

  // XCD-aware work mapping: all token ranges of one (layer, request, head pack)
  // land on the same XCD (blockIdx % 8), so its query tiles are fetched from HBM
  // into that XCD's L2 once.  With several requests the grid is sized for the
  // longest, so the ranges past a shorter request's end are empty and its last one
  // partial; each pair then takes its ranges in an order rotated by its place on
  // the XCD, which spreads the empty and partial ones over the dispatch positions.
  // In plain order range c always sits at position c mod 4 of the XCD's sequence,
  // and with 8 ranges per pair the positions holding ranges 0 and 4 then carry
  // most of the work (36 layers x 8 requests of 13103-58038 tokens: 9.29 ms plain,
  // 8.65 ms rotated; uniform lengths in a table padded to 8 ranges: 10.9 ms plain,
  // 9.0 ms rotated).  One request keeps the plain order (36 x 32768 tokens:
  // 1.044 ms plain, 1.061 ms rotated).
  const int bid = blockIdx.x;
  const int xcd = bid & 7, jj = bid >> 3;
  const int p = (jj / cpp) * 8 + xcd;
  const int chunk = a.R > 1 ? (jj + jj / cpp) % cpp : jj % cpp;
  if (p >= pairs) return;
  const int hpk = a.Hkv / HP;           // head packs per (layer, request)
  const int h0 = (p % hpk) * HP;
  const int r = (p / hpk) % a.R;
  const int l = p / (hpk * a.R);
  const int S = seq_len_of(a, r);
  const int t_begin = chunk * tpw;
  if (t_begin >= S) return;
  const int t_end = min(t_begin + tpw, S);
  const int nq_all = a.n_valid ? min(max(a.n_valid[r], 0), a.N) : a.N;
  const int nq = min(max(nq_all - a.qc0, 0), a.qcn);
  if (nq <= 0) return;
  const int n0 = a.n_seen[r] + min(nq_all, a.qc0);
  const int BS = a.BS;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lcol = lane & 31, lh = lane >> 5;
  const int rg = wave % RG, tg = wave / RG;
  const int hi = rg / RGH, rgl = rg % RGH;   // this wave's head in the pack, row group within it
  const int h = h0 + hi;
  const bool active = rgl * 64 < nq * G;  // this wave's rows hold at least one query row

  // ---- set-up: every load goes out before the first wait
  const int b0 = t_begin >> bs_shift;
  const int nbt = ((t_end - 1) >> bs_shift) - b0 + 1;  // <= 512: one entry per thread
  const int bt_own = a.bt[(int64_t)r * a.bt_sr + b0 + min(tid, nbt - 1)];
  V8 af[2][KS];
  f32x16 seed[2];
  int lim[2][4][QG];
  {
    const T *qbase = (const T *)a.q + (int64_t)l * a.q_sl + (int64_t)r * a.q_sr;
    const float *lbase = a.lse + (int64_t)l * a.lse_sl + (int64_t)r * a.lse_sr;
    const float inv_scale = 1.0f / a.scale;
    // rows are laid out by G, the group size padded to 1, 2, 4 or 8; a.G <= G is the
    // model's own (query head h * a.G + g): rows with g >= a.G are padding, a zero query
    // with seed -inf, so they never win the max over the group
    const int GR = a.G;
    // unconditional loads at clamped rows: no branch serialises them
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) {
      const int row = rgl * 64 + jt * 32 + lcol;
      const int n = row / G, g = row % G;
      const T *qp = qbase + (int64_t)(a.qc0 + min(n, nq - 1)) * a.q_sn + (int64_t)(h * GR + min(g, GR - 1)) * a.q_sh +
                    lh * 8;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const V8 v = *(const V8 *)(qp + ks * 16);
        af[jt][ks] = n < nq && g < GR ? v : (V8)(T)0;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int rw = rgl * 64 + jt * 32 + 8 * i + 4 * lh + j;
          const int nn = rw / G, gg = rw % G;
          const float v = lbase[(int64_t)(a.qc0 + min(nn, nq - 1)) * a.lse_sn + h * GR + min(gg, GR - 1)];
          seed[jt][4 * i + j] = nn < nq && gg < GR ? -v * inv_scale : -INFINITY;
        }
        if constexpr (CAUSAL && G == 16) {
          // rows 16 q' .. 16 q' + 15 of the tile are one query (groups 2 q' and 2 q' + 1 of
          // both halves); this lane finishes query q' = lh
          if (i == 0) {
            const int nn = (rgl * 64 + jt * 32 + 16 * lh) / G;
            const int v = a.kv_len[(int64_t)r * a.N + a.qc0 + min(nn, nq - 1)];
            lim[jt][0][0] = nn < nq ? v : 0;
          } else {
            lim[jt][i][0] = 0;
          }
        } else if constexpr (CAUSAL && G == 8) {
          // rows 8 i' .. 8 i' + 7 of the tile are one query (heads 0-3 in lanes 0-31,
          // 4-7 in lanes 32-63); this lane finishes queries i' = 2 lh and 2 lh + 1
          if (i < 2) {
            const int nn = (rgl * 64 + jt * 32 + 8 * (2 * lh + i)) / G;
            const int v = a.kv_len[(int64_t)r * a.N + a.qc0 + min(nn, nq - 1)];
            lim[jt][i][0] = nn < nq ? v : 0;
          } else {
            lim[jt][i][0] = 0;
          }
        } else if constexpr (CAUSAL) {
#pragma unroll
          for (int qg = 0; qg < QG; ++qg) {
            const int nn = (rgl * 64 + jt * 32 + 8 * i + 4 * lh + qg * G) / G;
            const int v = a.kv_len[(int64_t)r * a.N + a.qc0 + min(nn, nq - 1)];
            lim[jt][i][qg] = nn < nq ? v : 0;
          }
        }
      }
    }
  }
  if (tid < nbt) bts[tid] = (bt_own >= 0 && bt_own < a.num_blocks) ? bt_own : -1;
  // every set-up load has landed: the chunk loop's counts of vector memory operations
  // start from zero, and no later wait for the query tile drains the chunk loads
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();

  const T *krow0 = (const T *)a.kv + (int64_t)l * a.kv_sl;
  const float c2 = a.scale * 1.4426950408889634f;
  float *obase0 = a.out + (int64_t)l * a.out_sl + (int64_t)r * a.out_sr + (int64_t)h0 * a.out_sh;
  const float fn0 = (float)n0, fden = (float)(n0 + nq);
  const int ld_tile = (wave * LPW) / KS, ld_ks = (wave * LPW) % KS;

  // Swizzled rows: a chunk in LDS is CH token rows of HROW bytes, the PB-byte pieces (256 at
  // head dim 128) of
  // heads h0 .. h0+HP-1 side by side, and each piece's 16-byte columns stored XOR-swizzled:
  // LDS column c of token t's piece holds that head's column c ^ (t % NC).  The chunk is
  // CHB / 16 units of 16 bytes; this wave's share is LPW loads of 64 consecutive units
  // (lane i of load j writes unit 64 (LPW wave + j) + i), so every load reads whole
  // PB-byte pieces, and with HP > 1 HP x PB contiguous bytes of each token's row.  A
  // token past t_end, or in a block the table marks invalid, reads row 0 of block 0
  // instead; its score is never written.
  auto load_chunk = [&](int cbase, unsigned char *kb) {
    const uint32_t dst = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_address(&kb[wave * LPW * 1024]));
    if constexpr (!SWZ) {
      // fragment layout: LPW B fragments of tile ld_tile, [tile][k step][lane] x 16 bytes
      const int t = cbase + ld_tile * 32 + lcol;
      const int bi = min((t >> bs_shift) - b0, nbt - 1);
      int phys = bts[bi];
      const bool ok = t < t_end && phys >= 0;
      phys = ok ? phys : 0;
      const int slot = ok ? (t & (BS - 1)) : 0;
      const T *kp = krow0 + (int64_t)h0 * a.kv_sh + (int64_t)phys * a.kv_sb + (int64_t)slot * a.kv_ss + lh * 8 +
                    ld_ks * 16;
#pragma unroll
      for (int i = 0; i < LPW; ++i) load_lds16(kp + i * 16, dst + i * 1024);
      return;
    }
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int u = (wave * LPW + i) * 64 + lane;   // 16-byte unit of the chunk
      const int tl = u / (HP * NC);                 // token of the chunk
      const int w = u % (HP * NC);
      const int hp = w >> NCS, col = (w & (NC - 1)) ^ (tl & (NC - 1));
      const int t = cbase + tl;
      const int bi = min((t >> bs_shift) - b0, nbt - 1);
      int phys = bts[bi];
      const bool ok = t < t_end && phys >= 0;
      phys = ok ? phys : 0;
      const int slot = ok ? (t & (BS - 1)) : 0;
      load_lds16(krow0 + (int64_t)phys * a.kv_sb + (int64_t)slot * a.kv_ss + (int64_t)(h0 + hp) * a.kv_sh + col * 8,
                 dst + i * 1024);
    }
  };
  // The running means of the HP x CH (head, token) pairs at cbase -> oldm[slot] (wave 0:
  // NOLD loads into LDS of 4 bytes per lane, at clamped in-range tokens; those past t_end
  // are not used).
  auto load_old = [&](int cbase, int slot) {
    if (wave == 0) {
      const uint32_t dst = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_address(&oldm[slot][0]));
#pragma unroll
      for (int i = 0; i < NOLD; ++i) {
        const int e = i * 64 + lane, eh = e / CH, et = e % CH;
        load_lds4(obase0 + (int64_t)eh * a.out_sh + min(cbase + et, t_end - 1), dst + i * 256);
      }
    }
  };
  // B operand of k step ks: lane (lcol, lh) takes token lcol's column 2 ks + lh of head hi,
  // at LDS column (2 ks + lh) ^ (lcol % 16) of its piece; any 16 consecutive lanes read 16
  // distinct columns (no bank conflict)
  int roff[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) roff[ks] = lcol * HROW + hi * PB + (((2 * ks + lh) ^ (lcol & (NC - 1))) << 4);
  auto read_b = [&](V8 (&b8)[KS], const unsigned char *kb, int tile) {
    if constexpr (SWZ) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) b8[ks] = *(const V8 *)(&kb[tile * 32 * HROW + roff[ks]]);
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) b8[ks] = *(const V8 *)(&kb[((tile * KS + ks) * 64 + lane) * 16]);
    }
  };
  auto mfma8 = [&](const V8 (&a8)[KS], const V8 (&b8)[KS], const f32x16 &c) {
    f32x16 acc = c;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (__is_same(T, __bf16))
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8[ks], b8[ks], acc, 0, 0, 0);
      else
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a8[ks], b8[ks], acc, 0, 0, 0);
    }
    return acc;
  };
  // exp/max/sum of one row tile at token t: sum over this lane's 16 rows
  auto post = [&](const f32x16 &acc, const int (&lm)[4][QG], int t) {
    float sum = 0.f;
    if constexpr (G == 16) {
      // query q' of the tile: groups 2 q' and 2 q' + 1 of this lane (8 heads) and of
      // lane +- 32 (the other 8); the swap gives both halves the max of all sixteen, and
      // half lh finishes query lh
      float m[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        float h8 = acc[8 * k];
#pragma unroll
        for (int e = 1; e < 8; ++e) h8 = vmax(h8, acc[8 * k + e]);
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(h8), __float_as_uint(h8), false, false);
        m[k] = vmax(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      }
      const float e = __builtin_amdgcn_exp2f((lh ? m[1] : m[0]) * c2);
      if constexpr (CAUSAL) sum += t < lm[0][0] ? e : 0.f;
      else sum += e;
      return sum;
    }
    if constexpr (G == 8) {
      // query i' of the tile: heads 0-3 in this lane's group i' (lanes 0-31), heads 4-7
      // in the same group of lane + 32; the symmetric swap gives both halves the max of
      // all eight, and each half finishes two of the four queries
      float m[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float h4 = vmax(vmax(acc[4 * i], acc[4 * i + 1]), vmax(acc[4 * i + 2], acc[4 * i + 3]));
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(h4), __float_as_uint(h4), false, false);
        m[i] = vmax(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      }
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const float e = __builtin_amdgcn_exp2f((lh ? m[2 + k] : m[k]) * c2);
        if constexpr (CAUSAL) sum += t < lm[k][0] ? e : 0.f;
        else sum += e;
      }
      return sum;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a0 = acc[4 * i], a1 = acc[4 * i + 1], a2 = acc[4 * i + 2], a3 = acc[4 * i + 3];
      if constexpr (G == 4) {
        const float e = __builtin_amdgcn_exp2f(vmax(vmax(a0, a1), vmax(a2, a3)) * c2);
        if constexpr (CAUSAL) sum += t < lm[i][0] ? e : 0.f;
        else sum += e;
      } else if constexpr (G == 2) {
        const float e0 = __builtin_amdgcn_exp2f(vmax(a0, a1) * c2);
        const float e1 = __builtin_amdgcn_exp2f(vmax(a2, a3) * c2);
        if constexpr (CAUSAL) sum += (t < lm[i][0] ? e0 : 0.f) + (t < lm[i][1] ? e1 : 0.f);
        else sum += e0 + e1;
      } else {
        const float v[4] = {a0, a1, a2, a3};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e = __builtin_amdgcn_exp2f(v[j] * c2);
          if constexpr (CAUSAL) sum += t < lm[i][j] ? e : 0.f;
          else sum += e;
        }
      }
    }
    return sum;
  };
  auto compute_chunk = [&](const unsigned char *kb, int buf, int cbase) {
    if (!active) {
#pragma unroll
      for (int k = 0; k < NT; ++k) red[buf][2 * rg + lh][(tg + k * TG) * 32 + lcol] = 0.f;
      return;
    }
    V8 bfa[KS], bfb[KS];
    read_b(bfa, kb, tg);
    f32x16 acc0, acc1;
    float s0 = 0.f, part[NT];
#pragma unroll
    for (int k = 0; k < NT; ++k) {
      const int tile = tg + k * TG;
      V8 (&cur)[KS] = (k & 1) ? bfb : bfa;
      V8 (&nxt)[KS] = (k & 1) ? bfa : bfb;
      acc0 = mfma8(af[0], cur, seed[0]);
      if (k > 0) part[k - 1] = s0 + post(acc1, lim[1], cbase + (tile - TG) * 32 + lcol);
      acc1 = mfma8(af[1], cur, seed[1]);
      if (k + 1 < NT) read_b(nxt, kb, tile + TG);
      s0 = post(acc0, lim[0], cbase + tile * 32 + lcol);
      // the first tile's fragment reads all go out before its first MFMA (left
      // unordered, each was issued and waited for just before its MFMA); chain 0
      // with the VALU work of the previous tile, chain 1 with the fragment reads
      // of the next tile and the VALU work of chain 0
      if (k == 0) __builtin_amdgcn_sched_group_barrier(0x100, KS, 0);   // DS read
#pragma unroll
      for (int i = 0; i < KS; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
        if (k > 0) __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU
      }
#pragma unroll
      for (int i = 0; i < KS; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (k + 1 < NT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    part[NT - 1] = s0 + post(acc1, lim[1], cbase + (tg + (NT - 1) * TG) * 32 + lcol);
    // stored after the loop: an LDS store waits for the chunk loads in flight
#pragma unroll
    for (int k = 0; k < NT; ++k) red[buf][2 * rg + lh][(tg + k * TG) * 32 + lcol] = part[k];
  };
  // thread (head eh, token et) of the first HP x CH adds that head's 2 RGH partial sums of
  // the token in a fixed order
  auto reduce_chunk = [&](int cbase, int buf, int slot) {
    if (tid < HP * CH) {
      const int eh = tid / CH, et = tid % CH;
      const int t = cbase + et;
      if (t < t_end && bts[(t >> bs_shift) - b0] >= 0) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 2 * RGH; ++i) s += red[buf][2 * RGH * eh + i][et];
        obase0[(int64_t)eh * a.out_sh + t] = (oldm[slot][tid] * fn0 + s) / fden;
      }
    }
  };

  // NBUF - 1 chunks in flight: step c waits for chunk c, hands it over with one barrier
  // and issues the loads of chunk c + NBUF - 1 (K into the buffer chunk c - 1 used, the
  // old means into ring slot (c + NBUF - 1) % 8, which no chunk still to be reduced
  // holds).  After the set-up every vector memory operation of the loop is a load into
  // LDS or a store: a wave issues LPW K loads per chunk, and wave 0 NOLD more for the old
  // means, after them.  Loads complete in issue order, so while any of chunk c's loads is
  // outstanding so are the (NBUF - 2) * LPW K loads of later chunks issued after it:
  // vmcnt((NBUF - 2) * LPW) means chunk c's share of this wave is in LDS.
  const int nch = (t_end - t_begin + CH - 1) / CH;
  constexpr int VMW = (NBUF - 2) * LPW;
  auto step = [&](int c, const unsigned char *kcur, unsigned char *knext) {
    const int cbase = t_begin + c * CH;
    lds_barrier<VMW>();   // chunk c is in LDS, every wave's share; chunk c-1 is finished
    if (c >= 1) reduce_chunk(cbase - CH, (c - 1) & 1, (c - 1) & 7);
    load_chunk(cbase + (NBUF - 1) * CH, knext);   // past the end: harmless in-bounds rows
    load_old(cbase + (NBUF - 1) * CH, (c + NBUF - 1) & 7);
    __builtin_amdgcn_sched_barrier(0);
    compute_chunk(kcur, c & 1, cbase);
    __builtin_amdgcn_sched_barrier(0);
  };
  load_chunk(t_begin, kbuf_a);
  load_old(t_begin, 0);
  if constexpr (NBUF >= 3) { load_chunk(t_begin + CH, kbuf_b); load_old(t_begin + CH, 1); }
  if constexpr (NBUF >= 4) { load_chunk(t_begin + 2 * CH, kbuf_c); load_old(t_begin + 2 * CH, 2); }
  if constexpr (NBUF == 2) {
    for (int c = 0; c < nch; c += 2) {
      step(c, kbuf_a, kbuf_b);
      if (c + 1 < nch) step(c + 1, kbuf_b, kbuf_a);
    }
  } else if constexpr (NBUF == 3) {
    for (int c = 0; c < nch; c += 3) {
      step(c, kbuf_a, kbuf_c);
      if (c + 1 < nch) step(c + 1, kbuf_b, kbuf_a);
      if (c + 2 < nch) step(c + 2, kbuf_c, kbuf_b);
    }
  } else {
    for (int c = 0; c < nch; c += 4) {
      step(c, kbuf_a, kbuf_d);
      if (c + 1 < nch) step(c + 1, kbuf_b, kbuf_a);
      if (c + 2 < nch) step(c + 2, kbuf_c, kbuf_b);
      if (c + 3 < nch) step(c + 3, kbuf_d, kbuf_c);
    }
  }
  lds_barrier<0>();     // no load into LDS outlives the workgroup; the last chunk is finished
  reduce_chunk(t_begin + (nch - 1) * CH, (nch - 1) & 1, (nch - 1) & 7);
}

__global__ void bump_n_seen_kernel(int32_t *n_seen, const int32_t *n_valid, int R, int N) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r < R) n_seen[r] += n_valid ? min(max(n_valid[r], 0), N) : N;
}

// Compute units of the current device (one query per device, cached).
static int device_cus() {
  static std::mutex mu;
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// Token range per workgroup of the K-slice kernel.  One workgroup fills a CU (its
// query tile takes most of the LDS), so the grid is sized in waves of CU-count
// workgroups: as many waves as keep every wave at least MIN_SLICES 32-token
// slices per wave of the workgroup, at most MAX_WAVES (each workgroup re-stages
// its query tile; fewer, larger workgroups amortise that), and the token range
// split evenly over the chunks of a pair.  A small problem -- one layer of one
// request -- thus still spreads over every CU.
static int kslice_tokens_per_wg(int pairs, int span, int nw) {
  constexpr int MIN_SLICES = 2, MAX_WAVES = 8, MAX_TOKENS = MFMA_MAX_TOKENS;
  const int64_t cus = device_cus();
  const int64_t spp = (span + 31) / 32;                       // slices per pair
  const int64_t total = (int64_t)pairs * spp;
  const int64_t waves = std::min<int64_t>(MAX_WAVES, std::max<int64_t>(1, total / (cus * nw * MIN_SLICES)));
  const int64_t padded = ((pairs + 7) / 8) * 8;               // pairs rounded to whole XCD groups
  const int64_t cpp = std::max<int64_t>(1, (waves * cus + padded - 1) / padded);
  const int64_t per = std::min<int64_t>(MAX_TOKENS / 32, (spp + cpp - 1) / cpp);
  return (int)(per * 32);
}

// Token range per workgroup of the query-tile kernel: a whole number of chunks.  One
// workgroup fills a CU, so the launch runs in rounds of CU-count workgroups, and
// each workgroup pays a set-up (block-table slice, query tile, first chunk) of
// about `setup` chunks before its pipeline runs.  The range minimises
// rounds x (setup + chunks per workgroup): one layer of one request spreads over
// every CU, 36 layers run 9 full rounds of 4096 tokens.
static int qreg_tokens_per_wg(int pairs, int span, int chunk, double setup) {
  const int64_t cus = device_cus();
  const int span_chunks = (span + chunk - 1) / chunk;
  const int max_chunks = std::min(span_chunks, MFMA_MAX_TOKENS / chunk);
  int best = 1;
  double best_cost = 0.0;
  for (int k = 1; k <= max_chunks; ++k) {
    const int64_t items = (int64_t)pairs * ((span_chunks + k - 1) / k);
    const double cost = (double)((items + cus - 1) / cus) * (setup + k);
    if (k == 1 || cost < best_cost) { best_cost = cost; best = k; }
  }
  return best * chunk;
}

// Which MFMA kernel scores a launch of `rows` query rows.  ACTKV_SCORE_KERNEL=qreg or
// kslice forces one of the two (both are exact; for timing and tests), read once.
enum MfmaChoice { MFMA_AUTO = 0, MFMA_QREG = 1, MFMA_KSLICE = 2 };
static int mfma_choice() {
  static const int c = [] {
    const char *e = getenv("ACTKV_SCORE_KERNEL");
    if (!e) return (int)MFMA_AUTO;
    if (!strcmp(e, "qreg")) return (int)MFMA_QREG;
    if (!strcmp(e, "kslice")) return (int)MFMA_KSLICE;
    return (int)MFMA_AUTO;
  }();
  return c;
}

template <typename T, typename V8, int G, int DH = 128>
static int launch_mfma(const ScoreArgs &a0, int bs_shift, hipStream_t st) {
  const int pairs = a0.L * a0.R * a0.Hkv;
  const int span = a0.max_blocks * a0.BS;
  const int q_per_launch = 512 / G;  // both kernels take at most 512 query rows
  const bool causal = a0.kv_len != nullptr;
  const int choice = mfma_choice();
  for (int qc0 = 0; qc0 < a0.N; qc0 += q_per_launch) {
    ScoreArgs a = a0;
    a.qc0 = qc0;
    a.qcn = std::min(q_per_launch, a0.N - qc0);
    const int rows = a.qcn * G;
    // measured on 36 layers x 4 x 8k (causal) and 36 x 32k: the query-register kernel
    // is faster up to 128 rows (several heads per workgroup: 4.6-4.9 TB/s of K against
    // 3.5-4.4) and above 384 (the matrix cores bound it); the K-slice kernel from 129 to
    // 384 rows (with 2 heads per workgroup, 4 row groups each, or 1 head and 4 row
    // groups, the query-register kernel took 4-10% longer there)
    // groups of 8 and 16 heads, and groups padded to 4, 8 or 16 (3, 5-7, 9-15), run on the
    // query-register kernel alone (one head per workgroup)
    const bool qreg = DH != 128 || G >= 8 || a0.G != G || choice == MFMA_QREG ||
                      (choice == MFMA_AUTO && (rows <= 128 || rows > 384));
    if (qreg) {
      // query tile in registers, K shared through LDS; RG row groups of 64 rows over HPV
      // heads per workgroup, chunks of CHV tokens, the first one's set-up costing about
      // SETUP chunks
#define ACTKV_QREG(RGV, NB, SW, CHV, SETUP, HPV)                                                   \
  do {                                                                                             \
    const int packs = a0.L * a0.R * (a0.Hkv / HPV);                                                \
    const int tpw = qreg_tokens_per_wg(packs, span, CHV, SETUP);                                   \
    const int cpp = (span + tpw - 1) / tpw;                                                        \
    const int grid = ((packs + 7) / 8) * 8 * cpp;                                                  \
    if (causal)                                                                                    \
      hipLaunchKernelGGL((score_qreg_kernel<T, V8, G, true, RGV, NB, SW, CHV, HPV, DH>), dim3(grid), \
                         dim3(512), 0, st, a, tpw, cpp, packs, bs_shift);                          \
    else                                                                                           \
      hipLaunchKernelGGL((score_qreg_kernel<T, V8, G, false, RGV, NB, SW, CHV, HPV, DH>), dim3(grid),\
                         dim3(512), 0, st, a, tpw, cpp, packs, bs_shift);                          \
  } while (0)
      // Up to 128 rows the call streams K at the HBM rate.  Several KV heads of the same
      // tokens then share a workgroup (8 up to 64 rows, 4 up to 128): every wave keeps 64
      // rows, and each token's K arrives as 4 or 8 contiguous 256-byte pieces (whole 2 KiB
      // rows with 8 heads of 128).  Measured on 36 layers x 4 x 8k, causal: 16 queries 491
      // against 532 us with one head per workgroup, 32 queries 530 against 580.  Above 384
      // rows the matrix cores bound it: fragment layout (fewer address instructions) and
      // two chunks in flight.  Set-up measured at ~5 us against ~3.7 us per 512-row chunk
      // of 128 tokens.
      if constexpr (G >= 8) {
        if (rows <= 128) ACTKV_QREG(2, 3, true, 128, 1.5, 1);
        else if (rows <= 256) ACTKV_QREG(4, 3, true, 128, 1.5, 1);
        else ACTKV_QREG(8, 2, false, 128, 1.5, 1);
      } else if (rows <= 64 && a0.Hkv % 8 == 0) ACTKV_QREG(8, 2, true, 32, 8.0, 8);
      else if (rows <= 128 && a0.Hkv % 4 == 0) ACTKV_QREG(8, 2, true, 64, 4.0, 4);
      else if (rows <= 128) ACTKV_QREG(2, 3, true, 128, 1.5, 1);
      else if (rows <= 256) ACTKV_QREG(4, 3, true, 128, 1.5, 1);
      else ACTKV_QREG(8, 2, false, 128, 1.5, 1);
#undef ACTKV_QREG
    } else {
      // 12 waves stream their own K slices against the tile in LDS, which keeps
      // more K in flight
      constexpr int NW = 12, TT = 1;
      const int tpw = kslice_tokens_per_wg(pairs, span, NW);
      const int cpp = (span + tpw - 1) / tpw;
      const int grid = ((pairs + 7) / 8) * 8 * cpp;
#define ACTKV_LAUNCH(ROWSV)                                                                        \
  do {                                                                                             \
    if (causal)                                                                                    \
      hipLaunchKernelGGL((score_kslice_kernel<T, V8, G, ROWSV, true, NW, TT>), dim3(grid),         \
                         dim3(NW * 64), 0, st, a, tpw, cpp, pairs, bs_shift);                      \
    else                                                                                           \
      hipLaunchKernelGGL((score_kslice_kernel<T, V8, G, ROWSV, false, NW, TT>), dim3(grid),        \
                         dim3(NW * 64), 0, st, a, tpw, cpp, pairs, bs_shift);                      \
  } while (0)
      if constexpr (G < 8 && DH == 128) {   // never reached otherwise (above)
        if (rows <= 128) ACTKV_LAUNCH(128);
        else if (rows <= 256) ACTKV_LAUNCH(256);
        else ACTKV_LAUNCH(512);
      }
#undef ACTKV_LAUNCH
    }
    int rc = actkv_check_launch();
    if (rc) return rc;
  }
  return ACTKV_OK;
}

// The group size laid out in rows (1, 2, 4, 8 or 16; groups in between are padded).
template <typename T, typename V8, int DH>
static int launch_mfma_groups(const ScoreArgs &a, int G, int bs_shift, hipStream_t st) {
  return G > 8 ? launch_mfma<T, V8, 16, DH>(a, bs_shift, st)
       : G > 4 ? launch_mfma<T, V8, 8, DH>(a, bs_shift, st)
       : G > 2 ? launch_mfma<T, V8, 4, DH>(a, bs_shift, st)
       : G == 2 ? launch_mfma<T, V8, 2, DH>(a, bs_shift, st)
                : launch_mfma<T, V8, 1, DH>(a, bs_shift, st);
}

template <typename QT, typename KT, int ROWS>
static int launch_generic_rows(const ScoreArgs &a, hipStream_t st) {
  const int span = a.max_blocks * a.BS;
  dim3 grid((span + 255) / 256, a.L * a.R * a.Hkv);
  const size_t shm = (size_t)(ROWS * a.D + 2 * ROWS) * sizeof(float);
  hipLaunchKernelGGL((score_generic_rows_kernel<QT, KT, ROWS>), grid, dim3(256), shm, st, a, std::min(a.G, ROWS));
  return actkv_check_launch();
}

template <typename QT, typename KT>
static int launch_generic(const ScoreArgs &a, hipStream_t st) {
  // head dims that are a multiple of 4 up to 512: query rows in chunks of at most 64, 32 or 16
  // rows (head dim up to 128, 256, 512: at most 32 KiB of LDS), and no more than the call's
  // N * G rows rounded up to a power of two (one action query of a small group, the
  // reference's per-token fold, computes no padding rows)
  if (a.D % 4 == 0 && a.D <= 512) {
    const int rmax = a.D <= 128 ? 64 : a.D <= 256 ? 32 : 16;
    const int64_t need = (int64_t)a.N * a.G;
    int rows = 1;
    while (rows < rmax && rows < need) rows *= 2;
    switch (rows) {
      case 1: return launch_generic_rows<QT, KT, 1>(a, st);
      case 2: return launch_generic_rows<QT, KT, 2>(a, st);
      case 4: return launch_generic_rows<QT, KT, 4>(a, st);
      case 8: return launch_generic_rows<QT, KT, 8>(a, st);
      case 16: return launch_generic_rows<QT, KT, 16>(a, st);
      case 32: return launch_generic_rows<QT, KT, 32>(a, st);
      default: return launch_generic_rows<QT, KT, 64>(a, st);
    }
  }
  const int span = a.max_blocks * a.BS;
  dim3 grid((span + 255) / 256, a.L * a.R * a.Hkv);
  const size_t shm = (size_t)(a.G * a.D + a.G) * sizeof(float);
  if (shm > 64 * 1024) return ACTKV_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((score_generic_kernel<QT, KT>), grid, dim3(256), shm, st, a);
  return actkv_check_launch();
}

template <typename QT>
static int dispatch_generic_kv(const ScoreArgs &a, int kv_dtype, hipStream_t st) {
  switch (kv_dtype) {
    case ACTKV_F32: return launch_generic<QT, float>(a, st);
    case ACTKV_F16: return launch_generic<QT, _Float16>(a, st);
    case ACTKV_BF16: return launch_generic<QT, __bf16>(a, st);
  }
  return ACTKV_ERR_INVALID_ARG;
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace actkv

using namespace actkv;

extern "C" int actkv_action_scores(
    const void *q, int q_dtype, int64_t q_sl, int64_t q_sr, int64_t q_sn, int64_t q_sh,
    const void *kv, int kv_dtype, int64_t kv_sl, int64_t kv_sb, int64_t kv_ss, int64_t kv_sh,
    int64_t num_blocks, const int32_t *block_table, int64_t bt_sr, int max_blocks,
    const int32_t *seq_used, const float *lse, int64_t lse_sl, int64_t lse_sr, int64_t lse_sn,
    float *out, int64_t out_sl, int64_t out_sr, int64_t out_sh, int64_t out_width,
    int32_t *n_seen, const int32_t *n_valid, const int32_t *kv_len, int L, int R, int N, int Hq,
    int Hkv, int D, int block_size, float scale, void *stream) {
  if (!q || !kv || !block_table || !seq_used || !lse || !out || !n_seen) return ACTKV_ERR_INVALID_ARG;
  if (L < 1 || R < 1 || N < 0 || Hq < 1 || Hkv < 1 || D < 1 || block_size < 1 || max_blocks < 1)
    return ACTKV_ERR_INVALID_ARG;
  if (Hq % Hkv != 0) return ACTKV_ERR_INVALID_ARG;
  if (out_width < (int64_t)max_blocks * block_size) return ACTKV_ERR_INVALID_ARG;
  if (dtype_size(q_dtype) == 0 || dtype_size(kv_dtype) == 0) return ACTKV_ERR_INVALID_ARG;
  if ((int64_t)max_blocks * block_size > 0x7fffffffLL) return ACTKV_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  if (N == 0) return ACTKV_OK;

  ScoreArgs a;
  a.q = q; a.q_sl = q_sl; a.q_sr = q_sr; a.q_sn = q_sn; a.q_sh = q_sh;
  a.kv = kv; a.kv_sl = kv_sl; a.kv_sb = kv_sb; a.kv_ss = kv_ss; a.kv_sh = kv_sh;
  a.num_blocks = num_blocks;
  a.bt = block_table; a.bt_sr = bt_sr; a.max_blocks = max_blocks;
  a.seq_used = seq_used;
  a.lse = lse; a.lse_sl = lse_sl; a.lse_sr = lse_sr; a.lse_sn = lse_sn;
  a.out = out; a.out_sl = out_sl; a.out_sr = out_sr; a.out_sh = out_sh;
  a.n_seen = n_seen; a.n_valid = n_valid; a.kv_len = kv_len;
  a.L = L; a.R = R; a.N = N; a.Hq = Hq; a.Hkv = Hkv; a.D = D; a.G = Hq / Hkv; a.BS = block_size;
  a.scale = scale; a.qc0 = 0; a.qcn = N;

  const int G = a.G;
  const bool vec_ok = aligned16(q) && aligned16(kv) && q_sl % 8 == 0 && q_sr % 8 == 0 &&
                      q_sn % 8 == 0 && q_sh % 8 == 0 && kv_sl % 8 == 0 && kv_sb % 8 == 0 &&
                      kv_ss % 8 == 0 && kv_sh % 8 == 0;
  // the MFMA path takes whole 16-token tiles from one block: power-of-two block sizes >= 16
  int bs_shift = -1;
  for (int sh = 4; sh < 31; ++sh)
    if (block_size == (1 << sh)) bs_shift = sh;
  const bool mfma_ok = q_dtype == kv_dtype && (kv_dtype == ACTKV_BF16 || kv_dtype == ACTKV_F16) &&
                       (D == 128 || D == 64) && G >= 1 && G <= 16 && scale > 0.f && vec_ok &&
                       bs_shift >= 0;
  int rc;
  if (mfma_ok) {
    if (kv_dtype == ACTKV_BF16)
      rc = D == 64 ? launch_mfma_groups<__bf16, bf16x8, 64>(a, G, bs_shift, st)
                   : launch_mfma_groups<__bf16, bf16x8, 128>(a, G, bs_shift, st);
    else
      rc = D == 64 ? launch_mfma_groups<_Float16, f16x8, 64>(a, G, bs_shift, st)
                   : launch_mfma_groups<_Float16, f16x8, 128>(a, G, bs_shift, st);
  } else {
    switch (q_dtype) {
      case ACTKV_F32: rc = dispatch_generic_kv<float>(a, kv_dtype, st); break;
      case ACTKV_F16: rc = dispatch_generic_kv<_Float16>(a, kv_dtype, st); break;
      default: rc = dispatch_generic_kv<__bf16>(a, kv_dtype, st); break;
    }
  }
  if (rc) return rc;
  hipLaunchKernelGGL(bump_n_seen_kernel, dim3((R + 255) / 256), dim3(256), 0, st, n_seen, n_valid,
                     R, N);
  return actkv_check_launch();
}
