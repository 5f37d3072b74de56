// Shared device helpers for the gfx950 kernels of the cached block-diffusion step.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "kernels.hpp"

namespace fdllm {

typedef uint16_t u16;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

enum DType : int { DT_BF16 = 0, DT_F16 = 1 };

constexpr int WAVE = 64;

// ---- scalar conversions (round to nearest even, as torch / cuBLAS casts do) -------------------
__device__ __forceinline__ float bf16_to_f32(u16 h) { return __uint_as_float(((uint32_t)h) << 16); }

// round to nearest even (v_cvt_pk_bf16_f32 on gfx950); NaN stays NaN
__device__ __forceinline__ u16 f32_to_bf16(float f) { return __builtin_bit_cast(u16, (__bf16)f); }

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
// two values rounded to the model dtype and packed (a in the low half), the same bits as two from_f32
// calls: bf16 by one v_cvt_pk_bf16_f32; fp16 by two scalar conversions, each behind an empty asm.  The
// conversions themselves agree bit for bit (packed or not), but an fp16 rounding of a product compiles
// either to an fp32 multiply and a conversion (two roundings) or to one mixed-precision fma
// (v_fma_mixlo_f16, one rounding); keeping the two values apart keeps the compiler's choice the same as
// for a lone from_f32, which is what the other kernels compile to
template <int DT> __device__ __forceinline__ uint32_t pack_f32x2(float a, float b) {
  if constexpr (DT == DT_BF16) {
    typedef float f32x2v __attribute__((ext_vector_type(2)));
    typedef __bf16 b16x2v __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v{a, b}), b16x2v));
  } else {
    u16 lo = f32_to_f16(a), hi = f32_to_f16(b);
    asm volatile("" : "+v"(lo));
    asm volatile("" : "+v"(hi));
    return (uint32_t)lo | ((uint32_t)hi << 16);
  }
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
// Sum / max over the four 16-lane rows of a wave (lanes l, l ^ 16, l ^ 32, l ^ 48), with the gfx950
// row-swap permutes (no LDS crossbar): permlane16_swap(x, x) yields the even and odd row of each row
// pair, permlane32_swap(x, x) the lower and upper half.
__device__ __forceinline__ float rows_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ float rows_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

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
// Taylor polynomial in Horner form with fused multiply-adds, and the 2^n scale applied exactly
// (ldexp; the same product as a multiply by 2^n built in the exponent field); 0 below -86 so nothing
// is subnormal.  Every operation is one IEEE fp32 op with
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
  // p * 2^n, exact: n >= -125 here, so 2^n and the product are normal
  return __builtin_ldexpf(p, (int)n);
}

// SiLU(gate) x up with the rounding points of _silu_fp32 (model/cuda.py:319-328): gate and up rounded to
// DT, silu = gate x (1 / (1 + exp(-gate))) in fp32 rounded to DT, the product rounded to DT.  The
// reciprocal is the hardware estimate refined by one Newton-Raphson step, r + r (1 - d r), which agrees
// with the IEEE quotient to within its last bit (the IEEE division sequence is several times as many
// instructions per element of an epilogue that is VALU work only); past 2^64 the estimate alone (the step
// would form inf x 0), for d = inf exactly 0.
template <int DT>
__device__ __forceinline__ u16 silu_mul(float g, float u) {
  const float gt = rnd<DT>(g), up = rnd<DT>(u);
  const float d = 1.0f + expf(-gt);
  float r = __builtin_amdgcn_rcpf(d);
  const float e = __builtin_fmaf(-d, r, 1.0f);
  r = d < 0x1p64f ? __builtin_fmaf(e, r, r) : r;
  const float sl = rnd<DT>(gt * r);
  return from_f32<DT>(sl * up);
}

// ---- agent-coherent exchange between workgroups of one launch ---------------------------------
// Each XCD has its own write-back L2, so data one workgroup hands to another inside a launch is
// written and read with agent-scope relaxed atomics (the sc1 cache policy: written through to memory,
// read past a possibly stale L2 line) instead of plain accesses plus a release fence, whose L2
// write-back costs ~20 us per launch on MI355X.  A writer waits for its stores to be acknowledged
// (s_waitcnt vmcnt(0)) before it signals.
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent4(f32x4* p, f32x4 v) {
  typedef unsigned long long u64;
  u64* q = reinterpret_cast<u64*>(p);
  __hip_atomic_store(q, __builtin_bit_cast(u64, f32x2_t{v[0], v[1]}), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(q + 1, __builtin_bit_cast(u64, f32x2_t{v[2], v[3]}), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x4 ld_agent4(const f32x4* p) {
  typedef unsigned long long u64;
  u64* q = reinterpret_cast<u64*>(const_cast<f32x4*>(p));
  f32x2_t lo = __builtin_bit_cast(f32x2_t, __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  f32x2_t hi = __builtin_bit_cast(f32x2_t, __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  return f32x4{lo[0], lo[1], hi[0], hi[1]};
}
__device__ __forceinline__ void wait_memory() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Split fix-up: returns true in every thread of the workgroup that arrived last of `expected`.
// Callers write their partials with st_agent* first; the last arriver reads them with ld_agent*.
// The counter is returned to zero, so the next launch starts clean.
// Loads and stores of data that other workgroups of the same launch write or read: with COH they are
// agent-scope (sc1) accesses, which always see the latest agent-visible value (a plain load may hit a
// stale line of this XCD's L2) and write through; without COH they are plain.
template <bool COH>
__device__ __forceinline__ u32x4 ld16(const void* p) {
  if constexpr (COH) {
    typedef unsigned long long u64;
    const u64* q = reinterpret_cast<const u64*>(p);
    const u64 a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const u64 b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return u32x4{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
  } else {
    return *reinterpret_cast<const u32x4*>(p);
  }
}
template <bool COH>
__device__ __forceinline__ void st16(void* p, u32x4 v) {
  if constexpr (COH) {
    typedef unsigned long long u64;
    u64* q = reinterpret_cast<u64*>(p);
    __hip_atomic_store(q, (u64)v[0] | ((u64)v[1] << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, (u64)v[2] | ((u64)v[3] << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *reinterpret_cast<u32x4*>(p) = v;
  }
}
template <bool COH>
__device__ __forceinline__ u32x2 ld8(const void* p) {
  if constexpr (COH) {
    typedef unsigned long long u64;
    const u64 a = __hip_atomic_load(reinterpret_cast<const u64*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return u32x2{(uint32_t)a, (uint32_t)(a >> 32)};
  } else {
    return *reinterpret_cast<const u32x2*>(p);
  }
}
template <bool COH>
__device__ __forceinline__ void st8(void* p, u32x2 v) {
  if constexpr (COH) {
    typedef unsigned long long u64;
    __hip_atomic_store(reinterpret_cast<u64*>(p), (u64)v[0] | ((u64)v[1] << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *reinterpret_cast<u32x2*>(p) = v;
  }
}
template <bool COH>
__device__ __forceinline__ float ldf(const float* p) {
  if constexpr (COH) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else return *p;
}
template <bool COH>
__device__ __forceinline__ void stf(float* p, float v) {
  if constexpr (COH) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}
template <bool COH>
__device__ __forceinline__ f32x4 ldf4(const f32x4* p) {
  const u32x4 v = ld16<COH>(p);
  return f32x4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
}
template <bool COH>
__device__ __forceinline__ f32x2_t ldf2(const float* p) {
  const u32x2 v = ld8<COH>(p);
  return f32x2_t{__uint_as_float(v[0]), __uint_as_float(v[1])};
}
template <bool COH>
__device__ __forceinline__ void stf2(float* p, f32x2_t v) {
  st8<COH>(p, u32x2{__float_as_uint(v[0]), __float_as_uint(v[1])});
}
template <bool COH>
__device__ __forceinline__ void stf4(f32x4* p, f32x4 v) {
  st16<COH>(p, u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])});
}

// Agent-coherent 16-byte accesses through a buffer resource (one instruction per lane with the sc1 cache
// policy, where the agent-scope atomics above take two 8-byte ones), addressed by a byte offset from a
// base that is uniform across the wave.
struct CohBuf {
  __amdgpu_buffer_rsrc_t r;
};
__device__ __forceinline__ CohBuf coh_buf(const void* base, unsigned bytes) {
  return CohBuf{__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000)};
}
constexpr int CPOL_SC1 = 16;
__device__ __forceinline__ f32x4 coh_ldf4(const CohBuf& b, unsigned off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(b.r, (int)off, 0, CPOL_SC1));
}
__device__ __forceinline__ f32x2_t coh_ldf2(const CohBuf& b, unsigned off) {
  return __builtin_bit_cast(f32x2_t, __builtin_amdgcn_raw_buffer_load_b64(b.r, (int)off, 0, CPOL_SC1));
}
__device__ __forceinline__ void coh_stf4(const CohBuf& b, unsigned off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), b.r, (int)off, 0, CPOL_SC1);
}
__device__ __forceinline__ void coh_stf2(const CohBuf& b, unsigned off, f32x2_t v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), b.r, (int)off, 0, CPOL_SC1);
}

// ---- group waits inside one launch (GroupWait, kernels.hpp) ----
// Workgroup i (linear index, any thread) zeroes counter i of the other bank when the previous launch used it.
__device__ __forceinline__ void group_clear_other(const GroupWait& gw, int i) {
  if (i < gw.clear)
    __hip_atomic_store(gw.cnt + (size_t)((1 - gw.bank) * GW_GROUPS + i) * GW_STRIDE, 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// The workgroup's stores are acknowledged, then it counts its arrival on group k and waits until all
// `members` have arrived.  Returns false in every thread when the wait timed out: the fault word is set
// and the caller skips the work that needed the group.  Wave 0 polls (uniform control flow: the count is
// read into a scalar register).
__device__ __forceinline__ bool group_arrive_wait(const GroupWait& gw, int k, unsigned members, int* lds_flag) {
  wait_memory();
  __syncthreads();
  unsigned* ctr = gw.cnt + (size_t)(gw.bank * GW_GROUPS + k) * GW_STRIDE;
  if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) == 0) {
    if (threadIdx.x == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const long long t0 = wall_clock64();
    int ok = 1;
    while (__builtin_amdgcn_readfirstlane(__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) < members) {
      if (wall_clock64() - t0 > gw.limit) {
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (threadIdx.x == 0) {
      if (!ok) __hip_atomic_store(gw.fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      *lds_flag = ok;
    }
  }
  __syncthreads();
  return *lds_flag != 0;
}

__device__ __forceinline__ bool arrive_last(unsigned* counter, unsigned expected, int* lds_flag) {
  wait_memory();
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int last = (old == expected - 1);
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *lds_flag = last;
  }
  __syncthreads();
  return *lds_flag != 0;
}

// ---- activations in MFMA-fragment order ---------------------------------------------------------
// A one-shot projection chain (at most 32 rows) keeps its activations (the residual stream, the
// attention output, SiLU * up) in the order its GEMMs load them: k step s (columns 32 s .. 32 s + 31)
// and row tile t (rows 16 t .. 16 t + 15) form one 1 KB block at element (2 s + t) x 512, whose 16 bytes
// at lane l = r % 16 + 16 g hold row 16 t + r % 16, columns 32 s + 8 g .. + 7 -- one MFMA operand
// fragment per block, so a wave's fragment load is one coalesced 1 KB read.  Element (r, c), r < 32:
__device__ __forceinline__ size_t frag_off(int r, int c) {
  return (size_t)((c >> 5) * 2 + (r >> 4)) * 512 + (size_t)((r & 15) + 16 * ((c >> 3) & 3)) * 8 + (c & 7);
}

// The large-M LDS-staged GEMM takes its (normalised) activations in the same 1 KB fragment blocks,
// ordered row block by row block: block (row block b, k step s) at element (b KS + s) x 512, KS k steps
// per row.  Element (r, c):
__device__ __forceinline__ size_t frag_blk_off(int r, int c, int KS) {
  return ((size_t)(r >> 4) * KS + (c >> 5)) * 512 + (size_t)((r & 15) + 16 * ((c >> 3) & 3)) * 8 + (c & 7);
}

// f(integral_constant<int, I>) for I = B .. E - 1, unrolled at compile time (register arrays indexed by
// I stay in registers)
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// ---- shift-down lane exchange --------------------------------------------------------------------
// lane_down<K>(v) returns, in lanes l < K, the value lane l + K holds (K a power of two up to 32; the
// other lanes get unspecified values): gfx950's permlane32 / permlane16 swaps for K = 32 / 16 and a DPP
// row shift within 16 lanes below that, none of them through LDS.  A reduction that applies it for
// K = 32, 16, ..., 1 leaves in lane 0 exactly the value the xor butterfly (__shfl_xor with 32, 16, ...,
// 1) leaves in every lane, since each lane it reads holds what the butterfly's lane of that index holds.
template <int K>
__device__ __forceinline__ unsigned lane_down(unsigned v) {
  static_assert(K == 1 || K == 2 || K == 4 || K == 8 || K == 16 || K == 32, "power of two up to 32");
  if constexpr (K == 32) {
    return __builtin_amdgcn_permlane32_swap(v, v, false, false)[1];
  } else if constexpr (K == 16) {
    return __builtin_amdgcn_permlane16_swap(v, v, false, false)[1];
  } else {
    return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x100 + K, 0xf, 0xf, false);  // row_shl:K
  }
}
template <int K>
__device__ __forceinline__ float lane_down(float v) { return __uint_as_float(lane_down<K>(__float_as_uint(v))); }
template <int K>
__device__ __forceinline__ int lane_down(int v) { return (int)lane_down<K>((unsigned)v); }

// ---- LDS helpers ---------------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_raw;

// One 16-byte global -> LDS copy per lane (gfx950 global_load_lds_dwordx4: a wave writes 1 KB at the
// wave-uniform LDS address, lane l at byte 16 l).  Kept out of kernel
// bodies: the builtin written in a kernel template's own body stops the host pass from emitting the
// kernel's launch stub.
__device__ __forceinline__ void lds_copy16(const u16* g, unsigned char* l) {
  __builtin_amdgcn_global_load_lds(g, (lds_raw*)l, 16, 0, 0);
}

// ds_read_b64_tr_b16 (gfx950 transposing LDS read: within each 16-lane group, lane q supplies 4 16-bit
// values at its address and lane m receives value m % 4 of lanes 4 (m / 4) .. + 3, i.e. one column of a
// 4 x 4 block per 16 lanes) written as inline asm.  The builtin form makes the compiler's wait-count pass
// wait for every outstanding global-to-LDS copy before the read (it cannot tell which LDS bytes a copy
// writes), which drains a copy pipeline on every block; in asm the read is invisible to that pass.  So the
// caller must (1) have waited for and published (barrier) the copies that wrote the bytes it reads, and
// (2) wait for the results with lds_wait() before using them.  `lds` is an LDS byte address.
template <int OFF = 0>
__device__ __forceinline__ u32x2 ds_read_tr16(uint32_t lds) {
  static_assert(OFF >= 0 && OFF < 65536, "16-bit immediate offset");
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(lds), "i"(OFF) : "memory");
  return r;
}
// ds_read_b128 in asm, for blocks of LDS reads the caller waits for at once (lds_wait): the compiler,
// left to itself, interleaves such reads with their MFMAs and waits for each pair (the whole LDS latency
// per pair).  Same contract as ds_read_tr16.
template <int OFF = 0>
__device__ __forceinline__ u32x4 ds_read16(uint32_t lds) {
  static_assert(OFF >= 0 && OFF < 65536, "16-bit immediate offset");
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(lds), "i"(OFF) : "memory");
  return r;
}
// Wait for every outstanding LDS read (lgkmcnt(0)) and make the registers v depend on the wait, so no use
// of them is scheduled above it.
template <typename V, int N>
__device__ __forceinline__ void lds_wait(V (&v)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i]));
}
// LDS byte address of a pointer into dynamic shared memory
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// s_waitcnt with the vector-memory count N (gfx9 encoding: vmcnt bits [3:0] and [15:14]; export and LDS
// counts left at their maxima, so only vector memory is waited for)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// ---- bf16/fp16 pairs packed in 32-bit words ---------------------------------------------------
template <int DT> __device__ __forceinline__ float lo_f32(uint32_t w) { return to_f32<DT>((u16)(w & 0xffffu)); }
template <int DT> __device__ __forceinline__ float hi_f32(uint32_t w) { return to_f32<DT>((u16)(w >> 16)); }
__device__ __forceinline__ uint32_t pack2(u16 a, u16 b) { return (uint32_t)a | ((uint32_t)b << 16); }

}  // namespace fdllm
