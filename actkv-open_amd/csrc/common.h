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

}  // namespace actkv

// Returns ACTKV_ERR_LAUNCH if the last launch failed.
static inline int actkv_check_launch() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? ACTKV_OK : ACTKV_ERR_LAUNCH;
}
