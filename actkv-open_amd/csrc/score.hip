// LSE-recovery scoring on a paged KV cache (ActKV Algorithm 3) for gfx950.
//
// Reference: actkv/kernels/lse_attn.py:85-163.  The reference launches one
// Triton program per (request, logical block, KV head) and folds ONE action
// query per launch, so K is re-read from HBM once per action token.  Here one
// workgroup owns a (layer, request, KV head, token range) work item, holds the
// whole action-query tile of that head (N queries x G group heads) in VGPRs as
// MFMA A-operands, and streams the head's K rows through LDS exactly once:
//
//   acc[row, t] = q_row . k_t - lse_row / scale            (bf16/fp16 MFMA, fp32 acc)
//   p[n, t]     = exp2(scale*log2(e) * max_g acc[(n,g), t]) (max over the GQA group
//                                                           before the exp: exp is monotonic)
//   sum[t]      = sum_n p[n, t]                              (lane shuffles + LDS)
//   out[t]      = (out[t] * n_seen + sum[t]) / (n_seen + nq) (== nq reference folds)
//
// The generic kernel covers every other shape/dtype (fp32 caches, head_dim not
// 128, group sizes other than 1/2/4) and follows the reference fold order
// exactly: for each query in turn, out += (p - out) / (n_seen + n + 1).
#include "common.h"

#include <algorithm>

namespace actkv {

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

// ------------------------------------------------------------------ MFMA tile
// One workgroup = WAVES waves; wave w holds rows [(w*RT)*16, (w*RT+RT)*16) of the
// [nq*G, 128] query tile as v_mfma_f32_16x16x32 A-operands (RT row tiles of 16
// rows = 16/G queries each).  K rows of the head stream through a
// double-buffered LDS stage of CH = 64 tokens (16 KiB), XOR-swizzled in 16-byte
// pieces so the B-operand reads (16 tokens x one piece) hit distinct banks.
//
// MFMA lane layout (16x16x32): lane L supplies A[L%16][8*(L/16)+j] and
// B[8*(L/16)+j][L%16] (j<8) and receives D[4*(L/16)+i][L%16] (i<4).  Rows are
// ordered (query, group head), so with G=4 a lane's four outputs are the four
// group heads of one query at one token: the GQA max is in-register.
template <typename T, typename V8, int G, int WAVES, int RT>
__global__ void __launch_bounds__(WAVES * 64) score_mfma_kernel(ScoreArgs a, int tpw, int cpp,
                                                                 int pairs) {
  constexpr int KS = 4, CH = 64, NT = WAVES * 64;  // head_dim 128 = KS x 32
  constexpr int QS = 4 / G;                    // queries per lane per row tile
  constexpr int PIECES = CH * 16;              // 16-byte pieces per stage
  constexpr int PPT = PIECES / NT;             // pieces per thread per stage
  static_assert(PIECES % NT == 0, "stage must divide evenly");
  __shared__ __attribute__((aligned(16))) unsigned char kbuf[2][CH * 256];
  __shared__ float red[2][WAVES][CH];

  // XCD-aware work mapping: all token chunks of one (layer, request, head)
  // pair land on the same XCD (blockIdx % 8), so its query tile is fetched
  // into that XCD's L2 once.
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

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lrow = lane & 15, lgrp = lane >> 4;
  const float c2 = a.scale * 1.4426950408889634f;
  const float inv_scale = 1.0f / a.scale;

  // ---- query tile -> A operands, -lse/scale -> accumulator seeds
  V8 qa[RT][KS];
  f32x4 cinit[RT];
  int lim[RT][QS];
  const T *qbase = (const T *)a.q + (int64_t)l * a.q_sl + (int64_t)r * a.q_sr;
  const float *lbase = a.lse + (int64_t)l * a.lse_sl + (int64_t)r * a.lse_sr;
#pragma unroll
  for (int jt = 0; jt < RT; ++jt) {
    const int row = (wave * RT + jt) * 16 + lrow;
    const int n = row / G, g = row % G;
    if (n < nq) {
      const T *qp = qbase + (int64_t)(a.qc0 + n) * a.q_sn + (int64_t)(h * G + g) * a.q_sh + lgrp * 8;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qa[jt][ks] = *(const V8 *)(qp + ks * 32);
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qa[jt][ks] = V8{};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int orow = (wave * RT + jt) * 16 + 4 * lgrp + i;
      const int on = orow / G, og = orow % G;
      cinit[jt][i] = on < nq ? -lbase[(int64_t)(a.qc0 + on) * a.lse_sn + h * G + og] * inv_scale : 0.f;
    }
#pragma unroll
    for (int qsl = 0; qsl < QS; ++qsl) {
      const int on = ((wave * RT + jt) * 16 + 4 * lgrp) / G + qsl;
      int lm = 0;
      if (on < nq) lm = a.kv_len ? a.kv_len[(int64_t)r * a.N + a.qc0 + on] : 0x7fffffff;
      lim[jt][qsl] = lm;
    }
  }

  // ---- K stage loader: piece e = tid + i*NT -> token e/16, piece e%16
  const T *kbase = (const T *)a.kv + (int64_t)l * a.kv_sl + (int64_t)h * a.kv_sh;
  const int32_t *btr = a.bt + (int64_t)r * a.bt_sr;
  uint4 pre[PPT];
  auto load_stage = [&](int cb) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int e = tid + i * NT;
      const int tk = e >> 4, pc = e & 15;
      const int t = cb + tk;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (t < t_end) {
        const int64_t phys = btr[t / a.BS];
        if (phys >= 0 && phys < a.num_blocks)
          v = *(const uint4 *)(kbase + phys * a.kv_sb + (int64_t)(t % a.BS) * a.kv_ss + pc * 8);
      }
      pre[i] = v;
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int e = tid + i * NT;
      const int tk = e >> 4, pc = e & 15;
      *(uint4 *)(&kbuf[buf][tk * 256 + ((pc ^ (tk & 15)) << 4)]) = pre[i];
    }
  };

  const int nchunks = (t_end - t_begin + CH - 1) / CH;
  load_stage(t_begin);
  store_stage(0);
  __syncthreads();

  float *obase = a.out + (int64_t)l * a.out_sl + (int64_t)r * a.out_sr + (int64_t)h * a.out_sh;
  const float fn0 = (float)n0, fden = (float)(n0 + nq);

  for (int c = 0; c < nchunks; ++c) {
    const int buf = c & 1;
    const int cb = t_begin + c * CH;
    if (c + 1 < nchunks) load_stage(cb + CH);

    float psum[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int tk = tt * 16 + lrow;
      V8 kb[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        kb[ks] = *(const V8 *)(&kbuf[buf][tk * 256 + (((ks * 4 + lgrp) ^ (tk & 15)) << 4)]);
      f32x4 acc[RT];
#pragma unroll
      for (int jt = 0; jt < RT; ++jt) acc[jt] = cinit[jt];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int jt = 0; jt < RT; ++jt) {
          if constexpr (sizeof(T) == 2 && __is_same(T, __bf16))
            acc[jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[jt][ks], kb[ks], acc[jt], 0, 0, 0);
          else
            acc[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[jt][ks], kb[ks], acc[jt], 0, 0, 0);
        }
      }
      const int t = cb + tk;
      float s = 0.f;
#pragma unroll
      for (int jt = 0; jt < RT; ++jt) {
        if constexpr (G == 4) {
          const float m = fmaxf(fmaxf(acc[jt][0], acc[jt][1]), fmaxf(acc[jt][2], acc[jt][3]));
          const float e = __builtin_amdgcn_exp2f(m * c2);
          s += t < lim[jt][0] ? e : 0.f;
        } else if constexpr (G == 2) {
          const float e0 = __builtin_amdgcn_exp2f(fmaxf(acc[jt][0], acc[jt][1]) * c2);
          const float e1 = __builtin_amdgcn_exp2f(fmaxf(acc[jt][2], acc[jt][3]) * c2);
          s += (t < lim[jt][0] ? e0 : 0.f) + (t < lim[jt][1] ? e1 : 0.f);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float e = __builtin_amdgcn_exp2f(acc[jt][i] * c2);
            s += t < lim[jt][i] ? e : 0.f;
          }
        }
      }
      psum[tt] = s;
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      float v = psum[tt];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      if (lgrp == 0) red[buf][wave][tt * 16 + lrow] = v;
    }
    if (c + 1 < nchunks) store_stage(buf ^ 1);
    __syncthreads();
    if (tid < CH) {
      const int t = cb + tid;
      if (t < t_end) {
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) tot += red[buf][w][tid];
        const float old = obase[t];
        obase[t] = (old * fn0 + tot) / fden;
      }
    }
  }
}

__global__ void bump_n_seen_kernel(int32_t *n_seen, const int32_t *n_valid, int R, int N) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r < R) n_seen[r] += n_valid ? min(max(n_valid[r], 0), N) : N;
}

template <typename T, typename V8, int G>
static int launch_mfma(const ScoreArgs &a0, hipStream_t st) {
  const int pairs = a0.L * a0.R * a0.Hkv;
  const int span = a0.max_blocks * a0.BS;
  const int rows_max = 512;  // 8 waves x 4 row tiles x 16 rows; more rows spill VGPRs
  const int q_per_launch = rows_max / G;
  for (int qc0 = 0; qc0 < a0.N; qc0 += q_per_launch) {
    ScoreArgs a = a0;
    a.qc0 = qc0;
    a.qcn = std::min(q_per_launch, a0.N - qc0);
    const int rows = a.qcn * G;
    // token range per workgroup: enough workgroups to fill 256 CUs several
    // times over, at least 256 tokens so the query tile load is amortised.
    const int64_t total_tiles = (int64_t)pairs * ((span + 63) / 64);
    int tiles_per_wg = (int)std::max<int64_t>(4, (total_tiles + 2047) / 2048);
    int tpw = tiles_per_wg * 64;
    if (tpw > span) tpw = ((span + 63) / 64) * 64;
    const int cpp = (span + tpw - 1) / tpw;
    const int grid = ((pairs + 7) / 8) * 8 * cpp;
#define ACTKV_LAUNCH(WV, RTV)                                                               \
  hipLaunchKernelGGL((score_mfma_kernel<T, V8, G, WV, RTV>), dim3(grid), dim3(WV * 64), 0, st, \
                     a, tpw, cpp, pairs)
    if (rows <= 64) ACTKV_LAUNCH(4, 1);
    else if (rows <= 128) ACTKV_LAUNCH(4, 2);
    else if (rows <= 256) ACTKV_LAUNCH(4, 4);
    else ACTKV_LAUNCH(8, 4);
#undef ACTKV_LAUNCH
    int rc = actkv_check_launch();
    if (rc) return rc;
  }
  return ACTKV_OK;
}

template <typename QT, typename KT>
static int launch_generic(const ScoreArgs &a, hipStream_t st) {
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
  const bool mfma_ok = q_dtype == kv_dtype && (kv_dtype == ACTKV_BF16 || kv_dtype == ACTKV_F16) &&
                       D == 128 && (G == 1 || G == 2 || G == 4) && scale > 0.f && vec_ok;
  int rc;
  if (mfma_ok) {
    if (kv_dtype == ACTKV_BF16) {
      rc = G == 4 ? launch_mfma<__bf16, bf16x8, 4>(a, st)
         : G == 2 ? launch_mfma<__bf16, bf16x8, 2>(a, st)
                  : launch_mfma<__bf16, bf16x8, 1>(a, st);
    } else {
      rc = G == 4 ? launch_mfma<_Float16, f16x8, 4>(a, st)
         : G == 2 ? launch_mfma<_Float16, f16x8, 2>(a, st)
                  : launch_mfma<_Float16, f16x8, 1>(a, st);
    }
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
