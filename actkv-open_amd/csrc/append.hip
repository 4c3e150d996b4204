// Device append and slot map for the paged cache (gfx950).
//
// Reference: actkv/paged.py:76-84 (PagedKVCache.append) and :93-97 (slot_map).  The
// host allocator (the free-block stack, paged.py:67-74) stays on the host, where its
// order is defined; it hands the device the request's block table.  One launch then
// writes the new tokens of every layer, K and V planes, of any number of requests:
//   slot(t)  = table[t / block_size] * block_size + t % block_size   (paged.py:96-97)
//   kv[l, 0, slot(start + i)] = k[l, i].to(kv dtype), same for V     (paged.py:80-83)
// Threads move 16-byte chunks of destination rows (8 elements of one token, head and
// plane), converting the source dtype with round-to-nearest-even as
// torch's .to() does (conversions go through float, which is exact for the 16-bit
// types).  Rows are Hkv*D contiguous elements when the cache's head stride is D; the
// kernel takes the strides as given.  Shapes whose rows are not 16-byte aligned (D not
// a multiple of 8, odd strides) take the same kernel one element per chunk.
#include "common.h"

namespace actkv {

struct AppendArgs {
  void *kv;
  int kv_dtype;
  int64_t kv_sl, kv_sv, kv_sb, kv_ss, kv_sh;
  int64_t num_blocks;
  const void *k, *v;
  int src_dtype;
  int64_t k_sl, k_sn, k_sh, v_sl, v_sn, v_sh;
  int L, Hkv, D, R, BS;
  const int32_t *starts;   // [R] first logical position written
  const int32_t *counts;   // [R] tokens appended
  const int64_t *src_off;  // [R] source token offset of request r (k/v rows [L, sum n, ...])
  const int32_t *bt;       // [R, bt_sr] block tables
  int64_t bt_sr;
  int max_blocks;
  int32_t *bad;            // set to 1 when a destination block is missing or out of the pool
};

template <typename T, int VEC>
struct Chunk { T e[VEC]; };

template <typename ST, int VEC>
__device__ __forceinline__ Chunk<ST, VEC> load_chunk(const ST *src) {
  Chunk<ST, VEC> c;
  if constexpr (VEC == 1) {
    c.e[0] = *src;
  } else {
#pragma unroll
    for (int w = 0; w < (int)(sizeof(ST) * VEC / 16); ++w) ((uint4 *)c.e)[w] = ((const uint4 *)src)[w];
  }
  return c;
}

template <typename DT, typename ST, int VEC>
__device__ __forceinline__ void store_chunk(DT *dst, const Chunk<ST, VEC> &c) {
  Chunk<DT, VEC> o;
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    if constexpr (__is_same(DT, ST)) o.e[e] = c.e[e];
    else o.e[e] = (DT)(float)c.e[e];
  }
  if constexpr (VEC == 1) {
    *dst = o.e[0];
  } else {
#pragma unroll
    for (int w = 0; w < (int)(sizeof(DT) * VEC / 16); ++w) ((uint4 *)dst)[w] = ((const uint4 *)o.e)[w];
  }
}

// Workgroup shape, from a sweep on the 36-layer, 8 x 128-head bf16 append of ~6.7k tokens:
// small workgroups (8 tokens of one layer plane, 16 KB) stream best, 5.5 TB/s against 5.3
// for torch's contiguous copy of the same bytes; 16-64 tokens or 4-72 planes per
// workgroup, 2-8 rows in flight and non-temporal source loads were within 5% or slower.
constexpr int kTok = 8;      // tokens per workgroup (a power of two)
constexpr int kLP = 1;       // (layer, plane) pairs per workgroup
constexpr int kUnroll = 4;   // rows per thread per pass, all loaded before any is stored
static_assert((kTok & (kTok - 1)) == 0 && kTok <= 256, "kTok: a power of two up to 256");

// grid (ceil(total / kTok), ceil(2L / kLP)), 256 threads.  A workgroup writes the rows of
// kTok tokens in kLP (layer, plane) pairs, pair p = layer * 2 + plane.  The first kTok
// threads resolve their token's request, destination slot and source row once (into LDS).
// Threads own a fixed chunk column of a row (cw = min(chunks per row, 256) columns, 256 / cw
// rows per pass) and stream rows with kUnroll of them in flight; no division in the loop
// when a row has at most 256 chunks.
template <typename DT, typename ST, int VEC>
__global__ void __launch_bounds__(256) append_kernel(AppendArgs a, int64_t total) {
  __shared__ int64_t s_dst[kTok], s_src[kTok];
  const int64_t tok0 = (int64_t)blockIdx.x * kTok;
  const int ntok = (int)(total - tok0 < kTok ? total - tok0 : kTok);
  const int p0 = blockIdx.y * kLP;
  const int np = 2 * a.L - p0 < kLP ? 2 * a.L - p0 : kLP;
  const int tid = threadIdx.x;
  if (tid < ntok) {
    const int64_t tok = tok0 + tid;
    // which request: R is small, a linear walk over the prefix of counts
    int r = 0;
    int64_t base = 0;
    while (r + 1 < a.R && tok >= base + a.counts[r]) { base += a.counts[r]; ++r; }
    const int i = (int)(tok - base);
    const int t = a.starts[r] + i;
    const int b = t / a.BS;
    const int64_t phys = b < a.max_blocks ? (int64_t)a.bt[(int64_t)r * a.bt_sr + b] : -1;
    const bool ok = phys >= 0 && phys < a.num_blocks;
    if (!ok && a.bad) a.bad[0] = 1;
    s_dst[tid] = ok ? phys * a.kv_sb + (int64_t)(t % a.BS) * a.kv_ss : -1;
    s_src[tid] = a.src_off[r] + i;  // source token row
  }
  __syncthreads();
  const int cph = a.D / VEC;        // chunks per head
  const int cpr = a.Hkv * cph;      // chunks per row
  const int cw = cpr < 256 ? cpr : 256;
  const int rpp = 256 / cw;         // rows per pass
  const int tcol = tid % cw, trow = tid / cw;
  if (trow >= rpp) return;          // 256 % cw threads have no column
  const int nrows = np * kTok;      // row q: pair p0 + q / kTok, token q % kTok (< ntok)
  DT *db = (DT *)a.kv;
  const ST *kb = (const ST *)a.k, *vb = (const ST *)a.v;
  for (int col = tcol; col < cpr; col += 256) {
    const int h = col / cph, d0 = (col - h * cph) * VEC;
    const int64_t doff = (int64_t)h * a.kv_sh + d0;
    const int64_t koff = (int64_t)h * a.k_sh + d0, voff = (int64_t)h * a.v_sh + d0;
    for (int q0 = trow; q0 < nrows; q0 += rpp * kUnroll) {
      Chunk<ST, VEC> reg[kUnroll];
      int64_t dst[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int q = q0 + u * rpp;
        dst[u] = -1;
        const int pi = q / kTok, tk = q % kTok;
        if (q < nrows && tk < ntok) {
          const int pr = p0 + pi, l = pr >> 1, plane = pr & 1;
          const int64_t drow = s_dst[tk];
          if (drow >= 0) {
            dst[u] = drow + (int64_t)l * a.kv_sl + plane * a.kv_sv + doff;
            const int64_t srow = s_src[tk];
            const ST *src = plane == 0 ? kb + (int64_t)l * a.k_sl + srow * a.k_sn + koff
                                       : vb + (int64_t)l * a.v_sl + srow * a.v_sn + voff;
            reg[u] = load_chunk<ST, VEC>(src);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        if (dst[u] >= 0) store_chunk<DT, ST, VEC>(db + dst[u], reg[u]);
    }
  }
}

// slots of positions [start, start + n) of one request: table[t / bs] * bs + t % bs
__global__ void slot_map_kernel(const int32_t *table, int nblocks, int start, int n, int bs,
                                int64_t *out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int t = start + i;
  const int b = t / bs;
  out[i] = b < nblocks ? (int64_t)table[b] * bs + t % bs : -1;
}

template <typename DT, int VEC>
static int launch_append_src(const AppendArgs &a, int64_t total, hipStream_t st) {
  const int64_t gx = (total + kTok - 1) / kTok;
  const int gy = (2 * a.L + kLP - 1) / kLP;
  if (gx > 0x7fffffffLL || gy > 65535 || (int64_t)a.Hkv * a.D > 0x7fffffffLL) return ACTKV_ERR_UNSUPPORTED;
  dim3 grid((unsigned)gx, gy);
  switch (a.src_dtype) {
    case ACTKV_F32: hipLaunchKernelGGL((append_kernel<DT, float, VEC>), grid, dim3(256), 0, st, a, total); break;
    case ACTKV_F16: hipLaunchKernelGGL((append_kernel<DT, _Float16, VEC>), grid, dim3(256), 0, st, a, total); break;
    default: hipLaunchKernelGGL((append_kernel<DT, __bf16, VEC>), grid, dim3(256), 0, st, a, total); break;
  }
  return actkv_check_launch();
}

template <typename DT>
static int launch_append(const AppendArgs &a, int64_t total, bool vec, hipStream_t st) {
  return vec ? launch_append_src<DT, 8>(a, total, st) : launch_append_src<DT, 1>(a, total, st);
}

}  // namespace actkv

using namespace actkv;

extern "C" int actkv_append(void *kv, int kv_dtype, int64_t kv_sl, int64_t kv_sv, int64_t kv_sb,
                            int64_t kv_ss, int64_t kv_sh, int64_t num_blocks, const void *k,
                            const void *v, int src_dtype, int64_t k_sl, int64_t k_sn,
                            int64_t k_sh, int64_t v_sl, int64_t v_sn, int64_t v_sh, int L,
                            int Hkv, int D, int R, const int32_t *starts, const int32_t *counts,
                            const int64_t *src_off, int64_t total, const int32_t *block_table,
                            int64_t bt_sr, int max_blocks, int block_size, int32_t *bad,
                            void *stream) {
  if (!kv || !k || !v || !starts || !counts || !src_off || !block_table) return ACTKV_ERR_INVALID_ARG;
  if (L < 1 || Hkv < 1 || D < 1 || R < 1 || total < 0 || max_blocks < 1 || block_size < 1 ||
      num_blocks < 1)
    return ACTKV_ERR_INVALID_ARG;
  if (dtype_size(kv_dtype) == 0 || dtype_size(src_dtype) == 0) return ACTKV_ERR_INVALID_ARG;
  // 8 elements per thread where every row start is 16-byte aligned in both tensors
  // (a 16-byte chunk of the cache, 16 or 32 bytes of the source), else one element
  const int64_t de = (int64_t)dtype_size(kv_dtype), se = (int64_t)dtype_size(src_dtype);
  auto a16 = [](int64_t bytes) { return bytes % 16 == 0; };
  const bool vec = D % 8 == 0 && !((uintptr_t)kv & 15) && !((uintptr_t)k & 15) && !((uintptr_t)v & 15) &&
                   a16(kv_sl * de) && a16(kv_sv * de) && a16(kv_sb * de) && a16(kv_ss * de) &&
                   a16(kv_sh * de) && a16(k_sl * se) && a16(k_sn * se) && a16(k_sh * se) &&
                   a16(v_sl * se) && a16(v_sn * se) && a16(v_sh * se);
  if (total == 0) return ACTKV_OK;
  AppendArgs a;
  a.kv = kv; a.kv_dtype = kv_dtype; a.kv_sl = kv_sl; a.kv_sv = kv_sv; a.kv_sb = kv_sb;
  a.kv_ss = kv_ss; a.kv_sh = kv_sh; a.num_blocks = num_blocks;
  a.k = k; a.v = v; a.src_dtype = src_dtype;
  a.k_sl = k_sl; a.k_sn = k_sn; a.k_sh = k_sh; a.v_sl = v_sl; a.v_sn = v_sn; a.v_sh = v_sh;
  a.L = L; a.Hkv = Hkv; a.D = D; a.R = R; a.BS = block_size;
  a.starts = starts; a.counts = counts; a.src_off = src_off;
  a.bt = block_table; a.bt_sr = bt_sr; a.max_blocks = max_blocks; a.bad = bad;
  hipStream_t st = (hipStream_t)stream;
  switch (kv_dtype) {
    case ACTKV_F32: return launch_append<float>(a, total, vec, st);
    case ACTKV_F16: return launch_append<_Float16>(a, total, vec, st);
    default: return launch_append<__bf16>(a, total, vec, st);
  }
}

extern "C" int actkv_slot_map(const int32_t *table_row, int nblocks, int start, int n,
                              int block_size, int64_t *out, void *stream) {
  if (!table_row || !out || nblocks < 0 || start < 0 || n < 0 || block_size < 1) return ACTKV_ERR_INVALID_ARG;
  if (n == 0) return ACTKV_OK;
  hipLaunchKernelGGL(slot_map_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     table_row, nblocks, start, n, block_size, out);
  return actkv_check_launch();
}
