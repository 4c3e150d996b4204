// float32 reductions in the order of torch's CPU kernels, shared by the
// keep-mask and LRFU kernels.
//
// torch CPU sum order (aten SumKernel cascade_sum): for a reduction over n rows
// of an S-column block, the column's value is a cascade of 16-row blocks (level
// power 4) when the column lies in the vectorized body (torch_body_end), and the
// 4-way interleaved "row_sum" order for the other columns.
#pragma once

#include "common.h"

namespace actkv {

// torch multi_row_sum with level_power 4 (exact for n < 2^20).
template <typename F>
__device__ __forceinline__ float cascade_sum(F ld, int n, int first, int stride) {
  float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
  int i = 0;
  for (; i + 16 <= n;) {
    for (int j = 0; j < 16; ++j) acc0 = __fadd_rn(acc0, ld(first + (i + j) * stride));
    i += 16;
    acc1 = __fadd_rn(acc1, acc0);
    acc0 = 0.f;
    if ((i & (15 << 4)) == 0) {
      acc2 = __fadd_rn(acc2, acc1);
      acc1 = 0.f;
      if ((i & (15 << 8)) == 0) {
        acc3 = __fadd_rn(acc3, acc2);
        acc2 = 0.f;
      }
    }
  }
  for (; i < n; ++i) acc0 = __fadd_rn(acc0, ld(first + i * stride));
  acc0 = __fadd_rn(acc0, acc1);
  acc0 = __fadd_rn(acc0, acc2);
  acc0 = __fadd_rn(acc0, acc3);
  return acc0;
}

// torch row_sum: 4 interleaved cascades, leftover rows into the first, then
// ((p0 + p1) + p2) + p3.
template <typename F>
__device__ __forceinline__ float ilp4_sum(F ld, int n) {
  const int nilp = n / 4;
  float p0 = cascade_sum(ld, nilp, 0, 4);
  const float p1 = cascade_sum(ld, nilp, 1, 4);
  const float p2 = cascade_sum(ld, nilp, 2, 4);
  const float p3 = cascade_sum(ld, nilp, 3, 4);
  for (int i = nilp * 4; i < n; ++i) p0 = __fadd_rn(p0, ld(i));
  p0 = __fadd_rn(p0, p1);
  p0 = __fadd_rn(p0, p2);
  p0 = __fadd_rn(p0, p3);
  return p0;
}

// Columns [0, torch_body_end(S)) of an S-column reduction are in the vectorized body:
// whole 32-column blocks (four 8-lane vectors), or, in a row of 4-7 columns, one
// 4-column block.  The rest (1-3 columns, every remainder after the 32-column blocks)
// take row_sum.  Checked against torch 2.10's CPU mean for 1-80 columns and 2-64 rows,
// strided and contiguous; a contiguous single column of 16 or more rows (torch's inner
// reduction) takes another order and is not modelled.
__device__ __forceinline__ int torch_body_end(int S) { return S >= 8 ? (S & ~31) : (S >= 4 ? 4 : 0); }

template <typename F>
__device__ __forceinline__ float torch_sum(F ld, int n, bool body) {
  return body ? cascade_sum(ld, n, 0, 1) : ilp4_sum(ld, n);
}

__device__ __forceinline__ float nanmax(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}

}  // namespace actkv
