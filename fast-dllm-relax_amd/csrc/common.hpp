// Shared device helpers for the gfx950 kernels of the cached block-diffusion step.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fdllm {

typedef uint16_t u16;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

enum DType : int { DT_BF16 = 0, DT_F16 = 1 };

constexpr int WAVE = 64;

// ---- scalar conversions (round to nearest even, as torch / cuBLAS casts do) -------------------
__device__ __forceinline__ float bf16_to_f32(u16 h) { return __uint_as_float(((uint32_t)h) << 16); }

__device__ __forceinline__ u16 f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u16)0x7fc0;  // NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (u16)(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(u16 h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}

__device__ __forceinline__ u16 f32_to_f16(float f) {
  _Float16 v = (_Float16)f;
  u16 h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

template <int DT> __device__ __forceinline__ float to_f32(u16 h) {
  if constexpr (DT == DT_BF16) return bf16_to_f32(h); else return f16_to_f32(h);
}
template <int DT> __device__ __forceinline__ u16 from_f32(float f) {
  if constexpr (DT == DT_BF16) return f32_to_bf16(f); else return f32_to_f16(f);
}
// value rounded to the model dtype, kept in fp32
template <int DT> __device__ __forceinline__ float rnd(float f) { return to_f32<DT>(from_f32<DT>(f)); }

// ---- MFMA 16x16x32 (A: 16 x 32, B: 32 x 16, C: 16 x 16 fp32) ---------------------------------
// Lane l supplies A[l % 16][8 * (l / 16) + e] and B[8 * (l / 16) + e][l % 16], e = 0..7, and holds
// C[4 * (l / 16) + i][l % 16], i = 0..3.  A and B share the k assignment, so any consistent
// permutation of k inside a 32-wide step gives the same dot products.
template <int DT> __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == DT_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// ---- wave reductions ------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
  for (int k = 32; k >= 1; k >>= 1) v += __shfl_xor(v, k, WAVE);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  for (int k = 32; k >= 1; k >>= 1) v = fmaxf(v, __shfl_xor(v, k, WAVE));
  return v;
}

// ---- deterministic exp for the confidence reduction ------------------------------------------
// exp(x) for x <= 0: Cody-Waite reduction with ln2 split into a 16-bit head and a tail, a degree-7
// Taylor polynomial in Horner form with fused multiply-adds, and the 2^n scale built in the
// exponent field; 0 below -86 so nothing is subnormal.  Every operation is one IEEE fp32 op with
// contraction off, so the CPU restatement of the confidence reproduces it bit for bit.
__device__ __forceinline__ float fd_exp_neg(float x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  if (x < -86.0f) return 0.0f;
  const float log2e = 1.44269502162933349609375f;
  const float ln2_hi = 0.693145751953125f;
  const float ln2_lo = 1.428606765330187045e-06f;
  float n = __builtin_rintf(x * log2e);
  float r = __builtin_fmaf(n, -ln2_hi, x);
  r = __builtin_fmaf(n, -ln2_lo, r);
  float p = 1.98412701e-4f;
  p = __builtin_fmaf(p, r, 1.38888892e-3f);
  p = __builtin_fmaf(p, r, 8.33333377e-3f);
  p = __builtin_fmaf(p, r, 4.16666679e-2f);
  p = __builtin_fmaf(p, r, 1.66666672e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = (int)n;
  float scale = __uint_as_float((uint32_t)(ni + 127) << 23);
  return p * scale;
}

// ---- split-K fix-up: the last workgroup of a group to arrive reduces --------------------------
// Returns true in every thread of the workgroup that arrived last.  Writers publish their partials
// with a device-scope release before the arrival count; the last arriver acquires before reading.
// The counter returns to zero, so a later launch (or a graph replay) starts from a clean state.
__device__ __forceinline__ bool arrive_last(int* counter, int expected, int* lds_flag) {
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    int last = (old == expected - 1);
    if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *lds_flag = last;
  }
  __syncthreads();
  bool last = *lds_flag != 0;
  if (last) __threadfence();
  return last;
}

}  // namespace fdllm
