// Shared device/host helpers for the DSA HIP library (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dsa_capi.h"

namespace dsa {

// ---------------------------------------------------------------------------
// element types and MFMA operand vectors
// ---------------------------------------------------------------------------
typedef __bf16 bf16;
typedef _Float16 f16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Element traits: storage type <-> fp32, and the 16x16x32 MFMA for it.
template <typename T> struct Elem;

template <> struct Elem<bf16> {
  typedef bf16x8 v8;
  static __device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
  static __device__ __forceinline__ bf16 from_f32(float x) { return (bf16)x; }
  static __device__ __forceinline__ f32x4 mfma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // 32x32 output, k = 16: A lane l holds row l%32, k 8*(l/32) .. +7; B lane
  // l holds k 8*(l/32) .. +7 of column l%32; C register r of lane l is row
  // 8*(r/4) + 4*(l/32) + r%4, column l%32
  static __device__ __forceinline__ f32x16 mfma32(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Elem<f16> {
  typedef f16x8 v8;
  static __device__ __forceinline__ float to_f32(f16 x) { return (float)x; }
  static __device__ __forceinline__ f16 from_f32(float x) { return (f16)x; }
  static __device__ __forceinline__ f32x4 mfma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mfma32(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// 16-byte <-> 8-element vector reinterpretation.
template <typename V>
__device__ __forceinline__ V as_v8(u32x4 x) { return __builtin_bit_cast(V, x); }
template <typename V>
__device__ __forceinline__ u32x4 as_u4(V x) { return __builtin_bit_cast(u32x4, x); }

// v_mfma_f32_16x16x16 (bf16 / fp16): A lane l holds A[l%16][4*(l/16) + j],
// B lane l holds B[4*(l/16) + j][l%16], C register r holds C[4*(l/16) + r][l%16].
typedef short s16x4 __attribute__((ext_vector_type(4)));
template <typename T> struct Mfma16;
template <> struct Mfma16<bf16> {
  static __device__ __forceinline__ f32x4 run(s16x4 a, s16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma16<f16> {
  static __device__ __forceinline__ f32x4 run(s16x4 a, s16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c,
                                                 0, 0, 0);
  }
};

// max(x, 0) as one integer max on the bits: a negative float (-0.0
// included) is a negative int32.  Equal to fmaxf(x, 0.f) for every non-NaN
// x; fmaxf of an MFMA result is lowered with an extra canonicalising max.
__device__ __forceinline__ float relu_bits(float x) { return __int_as_float(max(__float_as_int(x), 0)); }

// Hardware exp2 (v_exp_f32); callers keep arguments <= 0 or -inf.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Butterfly max/sum across the four 16-lane groups that share lane%16, on
// the VALU lane-swap instructions of gfx950: v_permlane16_swap with both
// operands v returns (v[l], v[l ^ 16]) on every lane and v_permlane32_swap
// (v[l], v[l ^ 32]).  The pairs and their order match the __shfl_xor(16)
// then __shfl_xor(32) butterfly, which goes through the LDS crossbar
// (ds_swizzle / ds_bpermute) instead, so results are bit-identical.
__device__ __forceinline__ float xgroup_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xgroup_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Butterfly max/sum over all 64 lanes of a wave.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Workgroup barrier that orders LDS only.  __syncthreads() also fences
// global memory, which makes the compiler drain every outstanding global
// load (s_waitcnt vmcnt(0)) before the barrier and kills load/compute
// overlap; tiles staged through registers stay in flight across this one.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// LDS swizzles for token rows stored as 16-byte chunks (chunk c of token t
// is stored at c ^ swz(t), low four bits only).  Chosen by measurement on
// gfx950 (SQ_LDS_BANK_CONFLICT over the exact access patterns): the nope
// swizzle is conflict-free both for ds_read_b128 of 16 tokens x 4 chunk
// columns (the A fragment of K.Q^T) and for ds_read_b64_tr_b16 over 16 rows
// x 2 chunks (the V^T fragment); the simpler ((t & 7) << 1 | t >> 3 & 1)
// form costs the b128 reads a 2-way conflict.  Rope rows are 128 bytes (8
// chunks) and only read by ds_read_b128.  Both depend on t mod 16 only.
__device__ __forceinline__ int nope_swz(int tok) {
  return (((tok & 3) << 2) | (((tok >> 2) & 1) * 3)) ^ (((tok >> 3) & 1) << 1);
}
__device__ __forceinline__ int rope_swz(int tok) { return (tok >> 1) & 7; }

}  // namespace dsa

// ---------------------------------------------------------------------------
// host-side error plumbing shared by the C-ABI entry points
// ---------------------------------------------------------------------------
namespace dsa {
void set_error(const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);
// CUs of the current device (cached per device; 256 when it cannot be queried)
int device_cu_count();
// Test hooks set by dsa_set_test_flags (0 in normal use).
constexpr int kTestForceGlobalGather = 1;  // gather with 64-bit addresses even below 2 GiB
constexpr int kTestSmallBwdChunks = 2;     // backward rows in chunks of a 64 KiB workspace budget
constexpr int kTestKlGeneric = 4;          // the KL backward takes its generic path at every shape
constexpr int kTestFwdWide = 8;            // D = 512 forwards run sfa_fwd_kernel (no column split)
constexpr int kTestLiUnfused = 16;         // the indexer runs its scores and its top-k as two launches
constexpr int kTestLiNoPair = 32;          // two query rows per batch run the one-row score kernel
int test_flags();
}  // namespace dsa

#define DSA_CHECK_ARG(cond, ...)                                  \
  do {                                                            \
    if (!(cond)) {                                                \
      ::dsa::set_error(__VA_ARGS__);                              \
      return DSA_ERR_INVALID;                                     \
    }                                                             \
  } while (0)

#define DSA_CHECK_SUPPORTED(cond, ...)                            \
  do {                                                            \
    if (!(cond)) {                                                \
      ::dsa::set_error(__VA_ARGS__);                              \
      return DSA_ERR_UNSUPPORTED;                                 \
    }                                                             \
  } while (0)

#define DSA_HIP(expr)                                             \
  do {                                                            \
    hipError_t _e = (expr);                                       \
    if (_e != hipSuccess) return ::dsa::hip_fail(_e, #expr);      \
  } while (0)
