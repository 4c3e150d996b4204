// Shared device helpers for the gfx950 ActKV kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "actkv.h"

#define ACTKV_WAVE 64

namespace actkv {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Element loads to fp32 for the three cache dtypes.
template <int DT> struct Elem;
template <> struct Elem<ACTKV_F32> {
  typedef float T;
  static __device__ __forceinline__ float ld(const float *p) { return *p; }
};
template <> struct Elem<ACTKV_F16> {
  typedef _Float16 T;
  static __device__ __forceinline__ float ld(const _Float16 *p) { return (float)*p; }
};
template <> struct Elem<ACTKV_BF16> {
  typedef __bf16 T;
  static __device__ __forceinline__ float ld(const __bf16 *p) { return (float)*p; }
};

static inline size_t dtype_size(int dt) {
  return dt == ACTKV_F32 ? 4 : (dt == ACTKV_F16 || dt == ACTKV_BF16) ? 2 : 0;
}

// Order-preserving uint32 key of a float: a > b  <=>  key(a) > key(b).
// -0 is folded onto +0 (they compare equal) and every NaN maps above +inf,
// as torch.topk ranks NaN above all numbers.
__device__ __forceinline__ uint32_t float_key(float f) {
  if (f != f) return 0xFFFFFFFFu;
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// j-th (0-based) set bit of x; x must have more than j set bits.
__device__ __forceinline__ int select_bit(uint32_t x, int j) {
  int pos = 0;
  int c = __popc(x & 0xFFFFu);
  if (j >= c) { j -= c; x >>= 16; pos += 16; }
  c = __popc(x & 0xFFu);
  if (j >= c) { j -= c; x >>= 8; pos += 8; }
  c = __popc(x & 0xFu);
  if (j >= c) { j -= c; x >>= 4; pos += 4; }
  c = __popc(x & 0x3u);
  if (j >= c) { j -= c; x >>= 2; pos += 2; }
  c = (int)(x & 0x1u);
  if (j >= c) { pos += 1; }
  return pos;
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, ACTKV_WAVE);
  return v;
}

// Inclusive scan of a uint32 over the 64 lanes of a wave with DPP lane moves, which stay in
// the VALU (a shuffle is an LDS-pipe permute with LDS latency per step): shifts by 1, 2, 4
// and 8 lanes within each 16-lane row, then the last lane of rows 0 and 2 added into rows 1
// and 3, then lane 31 added into rows 2 and 3.  Lanes whose source is outside the row, or
// whose row the step leaves out, take `ident` (the identity of the associative `op`).
// Lane 63 ends with the whole wave's result.  Every lane of the wave must be active.
template <typename Op>
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t v, uint32_t ident, Op op) {
  const int id = (int)ident;
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x111, 0xf, 0xf, false));  // row_shr:1
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x112, 0xf, 0xf, false));  // row_shr:2
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x114, 0xf, 0xf, false));  // row_shr:4
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x118, 0xf, 0xf, false));  // row_shr:8
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x142, 0xa, 0xf, false));  // row_bcast:15
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x143, 0xc, 0xf, false));  // row_bcast:31
  return v;
}

struct OpAdd { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a + b; } };
struct OpMin { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a < b ? a : b; } };
struct OpMax { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; } };

// The whole wave's sum / min / max, in every lane.
__device__ __forceinline__ uint32_t wave_total_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readlane((int)wave_scan_u32(v, 0u, OpAdd()), 63);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readlane((int)wave_scan_u32(v, 0xFFFFFFFFu, OpMin()), 63);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readlane((int)wave_scan_u32(v, 0u, OpMax()), 63);
}

}  // namespace actkv

// Returns ACTKV_ERR_LAUNCH if the last launch failed.
static inline int actkv_check_launch() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? ACTKV_OK : ACTKV_ERR_LAUNCH;
}
