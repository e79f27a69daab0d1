// Helpers shared by the sparse and dense indexer KL-loss kernels.
#pragma once

#include "common.h"

namespace dsa {

// x = hi + mid + lo exactly (bf16 parts of an fp32 value: 8 + 8 + 8 bits),
// as the A operand of a 16x16x16 product whose k index is this lane's r
struct Split3 {
  s16x4 h, m, l;
};
__device__ __forceinline__ void split3_set(Split3& s, int r, float x) {
  const bf16 h = (bf16)x;
  const float r1 = x - (float)h;
  const bf16 m = (bf16)r1;
  const bf16 l = (bf16)(r1 - (float)m);
  s.h[r] = __builtin_bit_cast(short, h);
  s.m[r] = __builtin_bit_cast(short, m);
  s.l[r] = __builtin_bit_cast(short, l);
}
// sum over k of A[row][k] (rows = MFMA rows of the A operand), all 16
// output columns equal: B = ones
__device__ __forceinline__ f32x4 split3_rowsum(const Split3& s) {
  const short one = __builtin_bit_cast(short, (bf16)1.f);
  const s16x4 ones = {one, one, one, one};
  f32x4 c = Mfma16<bf16>::run(s.h, ones, (f32x4){0.f, 0.f, 0.f, 0.f});
  c = Mfma16<bf16>::run(s.m, ones, c);
  return Mfma16<bf16>::run(s.l, ones, c);
}

__device__ __forceinline__ float load_w(const void* w, int64_t i, int dt) {
  if (dt == DSA_DTYPE_FP32) return ((const float*)w)[i];
  if (dt == DSA_DTYPE_BF16) return (float)((const bf16*)w)[i];
  return (float)((const f16*)w)[i];
}

__device__ __forceinline__ void store_w(void* w, int64_t i, int dt, float v) {
  if (dt == DSA_DTYPE_FP32) ((float*)w)[i] = v;
  else if (dt == DSA_DTYPE_BF16) ((bf16*)w)[i] = (bf16)v;
  else ((f16*)w)[i] = (f16)v;
}

}  // namespace dsa
