// The cached block step (forward_cached / forward_block_partial_rp*, fast_dllm_relax/model/cuda.py:639-666,
// 723-788) for one sequence of at most 32 rows as ONE cooperative launch: every workgroup runs every
// layer, and the stages of a layer are separated by grid barriers instead of kernel boundaries.
//
//   per layer (cuda.py:561-579):
//     Q  qkv projection, RMSNorm on load, + bias               workgroups [0, qkv tiles)
//     A  RoPE, KV append, GQA attention over one key chunk     (query-tile group, kv head, chunk) units
//     M  merge of the key chunks (when there is more than one)  one wave per (16 dims, query tile, kv head)
//     O  o_proj + residual, row sums of squares                workgroups [0, hidden / 16)
//     U  gate_up, RMSNorm on load, SiLU(g) * u                  1 to 3 tile pairs per workgroup
//     D  down, k split across workgroups; the last of a tile group to arrive adds the splits in split
//        order + residual, row sums of squares
//
// What a launch boundary cannot do, a persistent workgroup does: the weights (and the cached K/V rows)
// of the NEXT stage do not depend on this stage's output, so each workgroup requests them into
// registers right after it has signalled the barrier and before it waits on it.  The HBM latency of
// the weight stream then overlaps the barrier instead of following it.
//
// Every stage runs the arithmetic of the per-operator kernels (the same k partition per wave, the same
// wave-order and split-order sums, the same epilogues and attention bodies), so the launch is bit-exact
// with the multi-kernel path for the same attention plan.
//
// Cross-workgroup data is written and read with agent-scope (sc1) accesses (common.hpp).  A barrier is
// one no-return atomic add per workgroup on one of 32 counters 128 B apart (after the workgroup's
// stores are acknowledged) and one wave per workgroup polling the 32 counters; every wait is bounded by
// a wall-clock deadline, after which the workgroup raises the abort flag and leaves, and every other
// workgroup leaves at its next wait.  The launch is cooperative, so all workgroups are co-resident.
#pragma once
#include "attn_body.hpp"
#include "gemm_body.hpp"

namespace fdllm {

// The same pointer, known to the compiler to be global memory (the parameters are read from memory, so
// their address space is otherwise unknown and every access would be a flat one, which also counts
// against the LDS counter).
template <typename T>
__device__ __forceinline__ T* gp(T* p) {
  return (T*)(__attribute__((address_space(1))) T*)(uintptr_t)p;
}

// ---- grid barrier ------------------------------------------------------------------------------
__device__ __forceinline__ unsigned ld_agent_u32(const unsigned* p) {
  return __hip_atomic_load(const_cast<unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Optional timeline: wall clock of this workgroup at (barrier n, slot) (slot 0 arrival, 1 release).
__device__ __forceinline__ void trace_at(const StepSync& s, unsigned n, int slot) {
  if (s.trace != nullptr && n < (unsigned)s.trace_bars)
    gp(s.trace)[((size_t)blockIdx.x * s.trace_bars + n) * 2 + slot] = wall_clock64();
}

// The workgroup has finished the stage before barrier n: its stores are acknowledged (every wave), then
// one arrival.
__device__ __forceinline__ void bar_arrive(const StepSync& s, unsigned n) {
  wait_memory();
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(gp(s.ctr) + BAR_STRIDE * (blockIdx.x % BAR_CTRS), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    trace_at(s, n, 0);
  }
}

// Wait until the n-th barrier (1-based) is complete: every workgroup has arrived n times.  Returns false
// (in every thread) when the launch is aborting.  Wave 0 polls; its loop is uniform control flow (the
// counter sum and the abort flag are read into scalar registers), so the values the other stages hold
// in registers across the wait are not copied around a divergent loop.
__device__ __forceinline__ bool bar_wait(const StepSync& s, unsigned n, int* lds_ok) {
  if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) == 0) {
    const unsigned lane = threadIdx.x;
    const unsigned target = n * gridDim.x;
    const long long t0 = wall_clock64();
    int ok = 1;
    while (true) {
      unsigned v = lane < BAR_CTRS ? ld_agent_u32(gp(s.ctr) + BAR_STRIDE * lane) : 0u;
      unsigned ab = lane == BAR_CTRS ? ld_agent_u32(gp(s.abort_f)) : 0u;
#pragma unroll
      for (int k = 32; k >= 1; k >>= 1) {
        v += __shfl_xor(v, k, WAVE);
        ab |= __shfl_xor(ab, k, WAVE);
      }
      if (__builtin_amdgcn_readfirstlane(v) >= target) break;
      if (__builtin_amdgcn_readfirstlane(ab) != 0u) { ok = 0; break; }
      if (wall_clock64() - t0 > s.limit) {
        if (lane == 0) {
          __hip_atomic_store(gp(s.abort_f), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(s.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) {
      *lds_ok = ok;
      trace_at(s, n, 1);
    }
  }
  __syncthreads();
  return *lds_ok != 0;
}

// ---- the launch's parameters ---------------------------------------------------------------------
static_assert(STEP_DNT == OsDownNT, "down groups are the one-shot kernel's");

// ---- register-resident weight blocks --------------------------------------------------------------
template <int NT, int KPW>
struct WBlocks {
  u32x4 A[KPW][NT];
};

// A copy of x the compiler cannot see through.  Every stage derives its lane indices and addresses
// from such a copy of threadIdx.x: otherwise the (loop-invariant) address arithmetic of all six stages
// is hoisted in front of the layer loop and held in registers across every stage.
__device__ __forceinline__ int opaque_v(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// this wave's share [ws, ws + wn) of kn k steps (the one-shot kernel's partition)
__device__ __forceinline__ void wave_ksplit(int kn, int w, int& ws, int& wn) {
  const int kq = kn / 8, kr = kn % 8;
  ws = kq * w + min(w, kr);
  wn = kq + (w < kr ? 1 : 0);
}

// Request the wave's blocks of tiles t[j] (j < nt), k steps kb + ws .. kb + ws + wn - 1 (wn >= 1) into
// registers.  Slots past wn repeat the last valid block (a cache hit) and are not multiplied.
template <int NT, int KPW>
__device__ __forceinline__ void w_issue(WBlocks<NT, KPW>& B, const u16* W, int KS, const int (&t)[NT], int nt, int kb,
                                        int ws, int wn, int lane) {
  const u32x4* base = reinterpret_cast<const u32x4*>(W) + lane;
#pragma unroll
  for (int s = 0; s < KPW; ++s)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      if (j < nt) B.A[s][j] = __builtin_nontemporal_load(base + ((size_t)t[j] * KS + kb + ws + min(s, wn - 1)) * 64);
    }
}

// Request the wave's blocks of tiles t[j] (j < nt), k steps kb + ws + s (s < wn) straight into LDS (the
// gfx950 global-to-LDS copy: one 1 KB block per instruction, lane l's 16 bytes at byte 16 l): block
// (s, j) lands at wbase + (s NT + j) KB.  A slice held in LDS occupies no registers while the workgroup
// waits at a barrier; the wave that requested it is the one that multiplies it, so a wait for its own
// memory counter is all the synchronisation it needs.
typedef __attribute__((address_space(3))) void lds_void;
template <int NT, int KPW>
__device__ __forceinline__ void w_issue_lds(unsigned char* wbase, const u16* W, int KS, const int (&t)[NT], int nt, int kb,
                                            int ws, int wn, int lane) {
  const u16* g = W + lane * 8;
#pragma unroll
  for (int s = 0; s < KPW; ++s)
#pragma unroll
    for (int j = 0; j < NT; ++j)
      if (s < wn && j < nt)
        __builtin_amdgcn_global_load_lds(g + ((size_t)t[j] * KS + kb + ws + s) * 512,
                                         (lds_void*)(wbase + (s * NT + j) * 1024), 16, 0, 0);
}

// The activation fragments of a wave's k steps: x[s][mt] holds rows 16 mt + (lane & 15) (rows past M
// repeat row M - 1), columns 32 (kb + ws + s) + 8 (lane >> 4) .. + 7, the MFMA B operand of k step s.
// Each wave multiplies only its own k steps, so it loads its slice of the rows straight into registers
// (agent-scope: other workgroups of the launch wrote them); nothing goes through LDS.
template <int KPW>
struct XFrags {
  u32x4 x[KPW][2];
};

// Agent-coherent loads through a buffer resource: one 16-byte (or 4-byte) load per lane with the sc1
// cache policy (a plain load may hit a stale line of this XCD's L2), addressed by a byte offset from a
// workgroup-uniform base.  (An agent-scope atomic load moves at most 8 bytes, so it would take twice the
// instructions.)
struct CohBuf {
  __amdgpu_buffer_rsrc_t r;
};
__device__ __forceinline__ CohBuf coh_buf(const void* base, unsigned bytes) {
  return CohBuf{__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000)};
}
constexpr int CPOL_SC1 = 16;
__device__ __forceinline__ u32x4 coh_ld16(const CohBuf& b, unsigned off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(b.r, (int)off, 0, CPOL_SC1));
}
__device__ __forceinline__ float coh_ldf(const CohBuf& b, unsigned off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(b.r, (int)off, 0, CPOL_SC1));
}

template <int KPW>
__device__ __forceinline__ void x_issue(XFrags<KPW>& X, const u16* src, int ldx, int M, int kb, int ws, int wn,
                                        int lane) {
  const CohBuf buf = coh_buf(src, (unsigned)((size_t)M * ldx * 2));
#pragma unroll
  for (int s = 0; s < KPW; ++s)
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int m = min(16 * mt + (lane & 15), M - 1);
      const int k = 32 * (kb + ws + min(s, wn - 1)) + 8 * (lane >> 4);
      X.x[s][mt] = coh_ld16(buf, (unsigned)(m * ldx + k) * 2u);
    }
}

// 1 / rms of the 32 rows (FastDLLMRMSNorm, cuda.py:269-275: mean of squares over the hidden width, from
// the per-16-column sums of squares the producer left) into inv_s: 8 threads per row, a fixed-order
// butterfly over the 8.  Ends with a workgroup barrier.
__device__ __forceinline__ void rms_inv(const float* ssq, int ssq_tiles, int ssq_ld, int M, int H, float eps,
                                        float* inv_s, int tid) {
  if (tid < 256) {
    const int m = tid >> 3, pp = tid & 7;
    const CohBuf buf = coh_buf(ssq, (unsigned)((size_t)ssq_tiles * ssq_ld * 4));
    float v[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int t = pp + 8 * q;
      v[q] = (m < M && t < ssq_tiles) ? coh_ldf(buf, (unsigned)(t * ssq_ld + m) * 4u) : 0.f;
    }
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < 16; ++q) ss += v[q];
    for (int q = 16; pp + 8 * q < ssq_tiles; ++q) ss += (m < M) ? coh_ldf(buf, (unsigned)((pp + 8 * q) * ssq_ld + m) * 4u) : 0.f;
    ss += __shfl_xor(ss, 1, WAVE);
    ss += __shfl_xor(ss, 2, WAVE);
    ss += __shfl_xor(ss, 4, WAVE);
    if (pp == 0) inv_s[m] = 1.0f / sqrtf(ss / (float)H + eps);
  }
  __syncthreads();
}

// x' = rnd(w[k] * rnd(x * inv_rms[m])) on the wave's fragments (gemm_os_body's XF_RMS transform).
template <int DT, int KPW>
__device__ __forceinline__ void x_norm(XFrags<KPW>& X, const u16* nw, int kb, int ws, int wn, const float* inv_s,
                                       int lane) {
  float inv[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) inv[mt] = inv_s[16 * mt + (lane & 15)];
#pragma unroll
  for (int s = 0; s < KPW; ++s) {
    const u32x4 wv = *reinterpret_cast<const u32x4*>(nw + 32 * (kb + ws + min(s, wn - 1)) + 8 * (lane >> 4));
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) X.x[s][mt] = xform<DT, XF_RMS>(X.x[s][mt], wv, inv[mt]);
  }
}

// The wave's products over its k steps: acc[t0 + j] += blocks B.A[.][bj0 + j] x X, j < nt (fp32 MFMA
// accumulation in k-step order, the one-shot kernel's).
template <int DT, int NTA, int NT, int KPW, int KX>
__device__ __forceinline__ void mfma_acc(f32x4 (&acc)[NTA][2], const WBlocks<NT, KPW>& B, int bj0, int t0, int nt, int wn,
                                         const XFrags<KX>& X) {
  static_assert(KX >= KPW, "fragments for every k step of the blocks");
#pragma unroll
  for (int s = 0; s < KPW; ++s)
    if (s < wn)
#pragma unroll
      for (int j = 0; j < NTA; ++j)
        if (j < nt)
#pragma unroll
          for (int mt = 0; mt < 2; ++mt) acc[t0 + j][mt] = mfma16<DT>(B.A[s][bj0 + j], X.x[s][mt], acc[t0 + j][mt]);
}

// mfma_acc with the weight blocks in LDS (laid out by w_issue_lds with NT tiles per k step).
template <int DT, int NTA, int NT, int KPW, int KX>
__device__ __forceinline__ void mfma_acc_lds(f32x4 (&acc)[NTA][2], const unsigned char* wbase, int bj0, int t0, int nt,
                                             int wn, const XFrags<KX>& X, int lane, int s0 = 0) {
  static_assert(KX >= KPW, "fragments for every k step of the blocks");
#pragma unroll
  for (int s = s0; s < KPW; ++s)
    if (s < wn)
#pragma unroll
      for (int j = 0; j < NTA; ++j)
        if (j < nt) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(wbase + (s * NT + bj0 + j) * 1024 + lane * 16);
#pragma unroll
          for (int mt = 0; mt < 2; ++mt) acc[t0 + j][mt] = mfma16<DT>(a, X.x[s][mt], acc[t0 + j][mt]);
        }
}

// The 8 waves' sums of tiles [0, nt) in LDS in wave order (gemm_os_body's step 5): on return, wave
// u < (nt / TPU) * 2 holds unit u = (tiles TPU (u / 2) .. + TPU - 1, row block u % 2) in v.
template <int TPU, int NT>
__device__ __forceinline__ void wave_sums(const f32x4 (&acc)[NT][2], int nt, unsigned char* smem, f32x4 (&v)[TPU],
                                          int tid) {
  constexpr int MT = 2;
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  __syncthreads();
  f32x4* red = reinterpret_cast<f32x4*>(smem);  // [8][NT][MT][64]
#pragma unroll
  for (int j = 0; j < NT; ++j)
    if (j < nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[((w * NT + j) * MT + mt) * 64 + lane] = acc[j][mt];
  __syncthreads();
  if (w < (nt / TPU) * MT) {
    const int ut = (w / MT) * TPU, umt = w % MT;
#pragma unroll
    for (int q = 0; q < TPU; ++q) {
      f32x4 sum = red[((0 * NT + ut + q) * MT + umt) * 64 + lane];
      for (int ww = 1; ww < 8; ++ww) sum += red[((ww * NT + ut + q) * MT + umt) * 64 + lane];
      v[q] = sum;
    }
  }
}

// One GEMM unit of a stage: the wave's products for its NT tiles (weights in LDS), then the wave sums.
// The LDS of the weights is reused for the sums (wave_sums waits for every wave first).
template <int DT, int TPU, int NT, int KPW>
__device__ __forceinline__ void mfma_reduce_lds(unsigned char* wbase, int nt, int wn, const XFrags<KPW>& X,
                                                unsigned char* smem, f32x4 (&v)[TPU], int tid) {
  f32x4 acc[NT][2];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j][0] = acc[j][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  wait_memory();  // this wave's global-to-LDS copies and its activation loads
  mfma_acc_lds<DT, NT, NT, KPW>(acc, wbase, 0, 0, nt, wn, X, tid & 63);
  wave_sums<TPU>(acc, nt, smem, v, tid);
}

// Copy of the scalar fields of an attention description (a whole copy would carry the per-sequence
// tables of a batched call, which a one-sequence launch never reads).
template <typename Src>
__device__ __forceinline__ void step_attn_view(const Src& s, AttnP& a) {
  a.qkv = gp(s.qkv); a.ldq = s.ldq; a.rows = s.rows; a.nq = s.nq; a.nkv = s.nkv; a.rope = gp(s.rope);
  a.kc = gp(s.kc); a.vc = gp(s.vc); a.ws = s.ws; a.Lk = s.Lk; a.scale = s.scale; a.mask = s.mask;
  a.q_pos0 = s.q_pos0; a.block = s.block; a.bias = s.bias; a.bias_ld = s.bias_ld; a.S = s.S; a.chunk = s.chunk;
  a.target_wgs = s.target_wgs; a.prefill_hpw = s.prefill_hpw; a.part = gp(s.part); a.out = gp(s.out); a.nseq = 1;
  a.seq_stride = 0;
  a.ofrag = 0;  // the persistent step keeps its activations row-major
}

// The launch's parameters are read through a constant-address-space pointer (scalar loads into scalar
// registers), and each stage re-reads them through a copy of that pointer the compiler cannot see
// through (see opaque_v), so that they are loaded where they are used instead of being held in
// registers across the whole kernel.
#define FD_CONSTANT __attribute__((address_space(4)))
template <typename T>
__device__ __forceinline__ const FD_CONSTANT T* opaque_c(const FD_CONSTANT T* x) {
  asm volatile("" : "+s"(x));
  return x;
}
template <typename T>
__device__ __forceinline__ const FD_CONSTANT T* as_constant(const T* x) {
  return (const FD_CONSTANT T*)(uintptr_t)x;
}

// LDS plan of a layer (bytes; KB = 1024).  Each slice is requested only after the workgroup's last access
// to the bytes it overwrites (bar_arrive synchronises the workgroup first):
//   Q  qkv slice [0, 48K), requested at the barrier before Q; its wave sums reuse [0, 16K)
//   A  K/V staging from 0
//   O  o_proj slice [0, 48K) and gate_up pair 0 [48K, 144K), both requested when A ends (pair 0 then
//      streams during the merge and o_proj stages); o_proj's wave sums at [0, 16K)
//   U  pair sums [0, 32K); pair 1's last k step [32K, 48K); wave 0's share of pair 1 [144K, 154K) (the
//      other waves hold theirs in registers)
//   D  down slice [0, 128K), requested when U ends; wave sums at [0, 64K)
// Wave 0 polls the barriers, so it requests nothing before a wait (its poll would otherwise wait for its
// own outstanding loads): wave 1 requests wave 0's blocks too, and a stage synchronises the workgroup
// before its waves read their slices.
constexpr int STEP_U_RK = STEP_KPW - 1;                                     // pair 1 k steps in registers
constexpr size_t STEP_LDS_U0 = (size_t)8 * STEP_KPW * 1024;                  // pair 0, past the o_proj slice
constexpr size_t STEP_LDS_U_P1L = (size_t)8 * 2 * 2 * 1024;                  // pair 1's last k step
constexpr size_t STEP_LDS_U_P1W0 = STEP_LDS_U0 + (size_t)8 * STEP_KPW * 2 * 1024;  // wave 0's pair 1
constexpr size_t STEP_LDS = STEP_LDS_U_P1W0 + (size_t)STEP_U_RK * 2 * 1024;
static_assert(STEP_LDS_U_P1L + (size_t)8 * (STEP_KPW - STEP_U_RK) * 2 * 1024 <= STEP_LDS_U0, "U plan");

// The barrier words of the launch (a copy out of the constant-space parameters).
template <typename S>
__device__ __forceinline__ StepSync sync_of(const S& s) {
  StepSync r;
  r.ctr = s.ctr; r.la = s.la; r.abort_f = s.abort_f; r.status = s.status; r.limit = s.limit;
  r.trace = s.trace; r.trace_bars = s.trace_bars;
  return r;
}

template <int DT, int CH>
__global__ __launch_bounds__(512) void step_kernel(StepP arg) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float inv_s[32];
  __shared__ int flag_s;
  const int b = blockIdx.x, G = gridDim.x;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // the argument is read in place in the kernel-argument segment (explicit arguments start at its
  // first byte), through a pointer each stage launders
  (void)arg;
  const FD_CONSTANT StepP* const pp = (const FD_CONSTANT StepP*)__builtin_amdgcn_kernarg_segment_ptr();
  const int L = pp->L;
  unsigned nbar = 0;  // barriers passed
  // the LDS slices of wave wv (see the LDS plan)
  auto slice_q = [&](int wv) { return smem + (size_t)wv * STEP_KPW * 1024; };
  auto slice_u0 = [&](int wv) { return smem + STEP_LDS_U0 + (size_t)wv * STEP_KPW * 2 * 1024; };
  auto slice_p1l = [&](int wv) { return smem + STEP_LDS_U_P1L + (size_t)wv * 2 * 1024; };
  auto slice_d = [&](int wv) { return smem + (size_t)wv * STEP_DKPW * STEP_DNT * 1024; };
  // a stage's requests into LDS before a barrier: every wave but 0 its own, wave 1 also wave 0's
  auto issue_waves = [&](auto&& issue_one) {
    if (w != 0) issue_one(w);
    if (w == 1) issue_one(0);
  };
  // this workgroup's qkv tile (b)
  auto q_issue = [&](int l) {
    auto& p = *opaque_c(pp);
    const int KS = p.H / 32, lane = opaque_v(threadIdx.x) & 63;
    const int t[1] = {b};
    issue_waves([&](int wv) {
      int ws, wn;
      wave_ksplit(KS, wv, ws, wn);
      w_issue_lds<1, STEP_KPW>(slice_q(wv), gp(as_constant(p.layers)[l].pqkv), KS, t, 1, 0, ws, wn, lane);
    });
  };
  // gate_up pairs of this workgroup: b, b + G, b + 2G
  auto u_pairs = [&](auto& p) { return b + 2 * G < p.np_u ? 3 : b + G < p.np_u ? 2 : b < p.np_u ? 1 : 0; };
  static_assert(STEP_PAIRS == 3, "the gate_up stage holds pair 0 in LDS, pair 1 in registers, pair 2 after pair 0");

  if (threadIdx.x == 0) trace_at(sync_of(pp->sync), 0, 0);
  if (b < pp->nt_q) q_issue(0);

  for (int l = 0; l < L; ++l) {
    // ---- Q: qkv = RMSNorm(h) . Wqkv^T + b ----
    {
      auto& p = *opaque_c(pp);
      if (b < p.nt_q) {
        const int tid = opaque_v(threadIdx.x), lane = tid & 63;
        const int KS = p.H / 32;
        int ws, wn;
        wave_ksplit(KS, w, ws, wn);
        auto& LW = as_constant(p.layers)[l];
        XFrags<STEP_KPW> X;
        x_issue(X, gp(p.h), p.H, p.M, 0, ws, wn, lane);
        rms_inv(gp(p.ssq), p.H / 16, p.ssq_ld, p.M, p.H, p.eps, inv_s, tid);
        x_norm<DT>(X, gp(LW.ln_in), 0, ws, wn, inv_s, lane);
        wait_memory();
        __syncthreads();  // wave 0's slice came from wave 1
        f32x4 v[1];
        mfma_reduce_lds<DT, 1, 1>(slice_q(w), 1, wn, X, smem, v, tid);
        if (w < 2) {
          GemmP g{};
          g.N = p.qkv_dim; g.M = p.M; g.Y = gp(p.qkv); g.ldy = p.qkv_dim; g.bias = gp(LW.bqkv);
          os_epilogue<DT, EPI_BIAS, 1, true>(g, v, 16 * w + (lane & 15), b, lane >> 4);
        }
      }
      bar_arrive(sync_of(p.sync), nbar + 1);
    }
    // the chunk's cached K/V rows do not depend on this layer's projection (wave 0 requests its share
    // after the wait)
    AttnChunkRegs<4, 2, CH> R;
    {
      auto& p = *opaque_c(pp);
      const int S = p.at.S;
      const bool has_a = b < p.qg * p.nkv * S;
      AttnP a;
      step_attn_view(p.at, a);
      a.kc = gp(p.kbase) + (size_t)l * p.layer_stride;
      a.vc = gp(p.vbase) + (size_t)l * p.layer_stride;
      if (has_a && w != 0) attn_chunk_load<4, 2, CH, true, CHUNK_CACHE>(a, (b / S) % p.nkv, b % S, R, opaque_v(threadIdx.x));
      if (!bar_wait(sync_of(p.sync), ++nbar, &flag_s)) return;
      if (has_a && w == 0) attn_chunk_load<4, 2, CH, true, CHUNK_CACHE>(a, (b / S) % p.nkv, b % S, R, opaque_v(threadIdx.x));
    }

    // ---- A: RoPE, KV append, attention over one key chunk ----
    {
      auto& p = *opaque_c(pp);
      const int S = p.at.S;
      if (b < p.qg * p.nkv * S) {
        const int tid = opaque_v(threadIdx.x);
        AttnP a;
        step_attn_view(p.at, a);
        a.kc = gp(p.kbase) + (size_t)l * p.layer_stride;
        a.vc = gp(p.vbase) + (size_t)l * p.layer_stride;
        const int ac = b % S, ag = (b / S) % p.nkv, aq = b / (S * p.nkv);
        attn_chunk_load<4, 2, CH, true, CHUNK_WINDOW>(a, ag, ac, R, tid);
        attn_chunk_compute<DT, 4, 2, CH, 0, true>(a, aq, ag, ac, smem, R, tid);
      }
      bar_arrive(sync_of(p.sync), nbar + 1);
      // o_proj's slice and gate_up pair 0, which then streams during the merge and o_proj stages
      const int lane = opaque_v(threadIdx.x) & 63;
      auto& LW = as_constant(p.layers)[l];
      if (b < p.nt_o) {
        const int KS = p.q_dim / 32;
        const int t[1] = {b};
        issue_waves([&](int wv) {
          int ws, wn;
          wave_ksplit(KS, wv, ws, wn);
          w_issue_lds<1, STEP_KPW>(slice_q(wv), gp(LW.po), KS, t, 1, 0, ws, wn, lane);
        });
      }
      if (u_pairs(p) > 0) {
        const int KS = p.H / 32;
        const int t[2] = {2 * b, 2 * b + 1};
        issue_waves([&](int wv) {
          int ws, wn;
          wave_ksplit(KS, wv, ws, wn);
          w_issue_lds<2, STEP_KPW>(slice_u0(wv), gp(LW.pgu), KS, t, 2, 0, ws, wn, lane);
        });
      }
      if (!bar_wait(sync_of(p.sync), ++nbar, &flag_s)) return;
    }

    // ---- M: merge of the key chunks ----
    {
      auto& p = *opaque_c(pp);
      if (p.at.S > 1) {
        const int QT = ((p.nq / p.nkv) * p.M + 15) / 16;
        const int u = b + G * w;
        if (u < 8 * QT * p.nkv) {
          AttnP a;
          step_attn_view(p.at, a);
          attn_merge_wave<DT, true>(a, u % 8, (u / 8) % QT, u / (8 * QT), opaque_v(threadIdx.x) & 63);
        }
        bar_arrive(sync_of(p.sync), nbar + 1);
        if (!bar_wait(sync_of(p.sync), ++nbar, &flag_s)) return;
      }
    }

    // ---- O: h += attn . Wo^T, row sums of squares ----
    WBlocks<2, STEP_U_RK> Bu;  // gate_up pair 1 but its last k step (waves 1..7)
    {
      auto& p = *opaque_c(pp);
      if (b < p.nt_o) {
        const int tid = opaque_v(threadIdx.x), lane = tid & 63;
        const int KS = p.q_dim / 32;
        int ws, wn;
        wave_ksplit(KS, w, ws, wn);
        XFrags<STEP_KPW> X;
        x_issue(X, gp(p.attn), p.q_dim, p.M, 0, ws, wn, lane);
        wait_memory();
        __syncthreads();  // wave 0's slice came from wave 1
        f32x4 v[1];
        mfma_reduce_lds<DT, 1, 1>(slice_q(w), 1, wn, X, smem, v, tid);
        if (w < 2) {
          GemmP g{};
          g.N = p.H; g.M = p.M; g.Y = gp(p.h); g.ldy = p.H; g.ssq_out = gp(p.ssq); g.ssq_ld = p.ssq_ld;
          os_epilogue<DT, EPI_RESID, 1, true>(g, v, 16 * w + (lane & 15), b, lane >> 4);
        }
      }
      bar_arrive(sync_of(p.sync), nbar + 1);
      if (u_pairs(p) > 1) {
        const int KS = p.H / 32, lane = opaque_v(threadIdx.x) & 63;
        auto& LW = as_constant(p.layers)[l];
        const int t[2] = {2 * (b + G), 2 * (b + G) + 1};
        if (w != 0) {
          int ws, wn;
          wave_ksplit(KS, w, ws, wn);
          w_issue(Bu, gp(LW.pgu), KS, t, 2, 0, ws, min(wn, STEP_U_RK), lane);
        }
        issue_waves([&](int wv) {
          int ws, wn;
          wave_ksplit(KS, wv, ws, wn);
          if (wv == 0)
            w_issue_lds<2, STEP_U_RK>(smem + STEP_LDS_U_P1W0, gp(LW.pgu), KS, t, 2, 0, ws, min(wn, STEP_U_RK), lane);
          if (wn > STEP_U_RK) w_issue_lds<2, 1>(slice_p1l(wv), gp(LW.pgu), KS, t, 2, 0, ws + STEP_U_RK, 1, lane);
        });
      }
      if (!bar_wait(sync_of(p.sync), ++nbar, &flag_s)) return;
    }

    // ---- U: act = SiLU(g) * u of RMSNorm(h) . Wgu^T ----
    {
      auto& p = *opaque_c(pp);
      const int up = u_pairs(p);
      if (up > 0) {
        const int tid = opaque_v(threadIdx.x), lane = tid & 63;
        const int KS = p.H / 32;
        int ws, wn;
        wave_ksplit(KS, w, ws, wn);
        auto& LW = as_constant(p.layers)[l];
        XFrags<STEP_KPW> X;
        x_issue(X, gp(p.h), p.H, p.M, 0, ws, wn, lane);
        rms_inv(gp(p.ssq), p.H / 16, p.ssq_ld, p.M, p.H, p.eps, inv_s, tid);
        x_norm<DT>(X, gp(LW.ln_post), 0, ws, wn, inv_s, lane);
        wait_memory();
        __syncthreads();  // wave 0's slices came from wave 1
        // one pair at a time (its two tiles' accumulators only), summed over the waves at [0, 32K);
        // waves 0 and 1 (row blocks) run the SiLU * up epilogue
#pragma unroll
        for (int k = 0; k < STEP_PAIRS; ++k) {
          if (k < up) {
            f32x4 acc[2][2];
            acc[0][0] = acc[0][1] = acc[1][0] = acc[1][1] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (k == 0) {
              mfma_acc_lds<DT, 2, 2, STEP_KPW>(acc, slice_u0(w), 0, 0, 2, wn, X, lane);
              if (up > 2) {
                // the third pair goes to the wave's pair-0 slice once the wave has read pair 0 from it
                wait_memory();
                const int t[2] = {2 * (b + 2 * G), 2 * (b + 2 * G) + 1};
                w_issue_lds<2, STEP_KPW>(slice_u0(w), gp(LW.pgu), KS, t, 2, 0, ws, wn, lane);
              }
            } else if (k == 1) {
              if (w != 0) mfma_acc<DT>(acc, Bu, 0, 0, 2, min(wn, STEP_U_RK), X);
              else mfma_acc_lds<DT, 2, 2, STEP_U_RK>(acc, smem + STEP_LDS_U_P1W0, 0, 0, 2, min(wn, STEP_U_RK), X, lane);
              // the last k step: block (0, j) of the wave's pair-1 LDS slice, with fragments of that step
              mfma_acc_lds<DT, 2, 2, STEP_KPW>(acc, slice_p1l(w) - (size_t)STEP_U_RK * 2 * 1024, 0, 0, 2, wn, X, lane,
                                               STEP_U_RK);
            } else {
              wait_memory();
              mfma_acc_lds<DT, 2, 2, STEP_KPW>(acc, slice_u0(w), 0, 0, 2, wn, X, lane);
            }
            f32x4 v[2];
            wave_sums<2>(acc, 2, smem, v, tid);
            if (w < 2) {
              GemmP g{};
              g.N = p.I; g.M = p.M; g.Y = gp(p.act); g.ldy = p.I;
              os_epilogue<DT, EPI_SILU_PAIR, 2, true>(g, v, 16 * w + (lane & 15), 2 * (b + k * G), lane >> 4);
            }
          }
        }
      }
      bar_arrive(sync_of(p.sync), nbar + 1);
      if (b < p.d_groups * p.d_splits) {
        const int dkps = p.I / 32 / p.d_splits, dgrp = b / p.d_splits, dsplit = b % p.d_splits;
        const int lane = opaque_v(threadIdx.x) & 63;
        int t[STEP_DNT];
#pragma unroll
        for (int j = 0; j < STEP_DNT; ++j) t[j] = dgrp * STEP_DNT + j;
        issue_waves([&](int wv) {
          int ws, wn;
          wave_ksplit(dkps, wv, ws, wn);
          w_issue_lds<STEP_DNT, STEP_DKPW>(slice_d(wv), gp(as_constant(p.layers)[l].pd), p.I / 32, t, STEP_DNT,
                                           dsplit * dkps, ws, wn, lane);
        });
      }
      if (!bar_wait(sync_of(p.sync), ++nbar, &flag_s)) return;
    }

    // ---- D: split partial of act . Wd^T; the group's last arriver adds the splits + residual ----
    {
      auto& p = *opaque_c(pp);
      if (b < p.d_groups * p.d_splits) {
        const int tid = opaque_v(threadIdx.x), lane = tid & 63;
        const int dkps = p.I / 32 / p.d_splits, dgrp = b / p.d_splits, dsplit = b % p.d_splits;
        int ws, wn;
        wave_ksplit(dkps, w, ws, wn);
        XFrags<STEP_DKPW> X;
        x_issue(X, gp(p.act), p.I, p.M, dsplit * dkps, ws, wn, lane);
        wait_memory();
        __syncthreads();  // wave 0's slice came from wave 1
        f32x4 v[1];
        mfma_reduce_lds<DT, 1, STEP_DNT>(slice_d(w), STEP_DNT, wn, X, smem, v, tid);
        constexpr int per = STEP_DNT * 2 * 64;
        f32x4* part = reinterpret_cast<f32x4*>(gp(p.dpart)) + ((size_t)dgrp * p.d_splits + dsplit) * per;
        stf4<true>(part + w * 64 + lane, v[0]);  // unit w = (tile w / 2, row block w % 2): the one-shot layout
        wait_memory();
        __syncthreads();
        if (tid == 0) {
          const unsigned old = __hip_atomic_fetch_add(gp(p.sync.la) + BAR_STRIDE * dgrp, 1u, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
          flag_s = old == (unsigned)((l + 1) * p.d_splits - 1);
        }
        __syncthreads();
        if (flag_s) {
          GemmP g{};
          g.N = p.H; g.M = p.M; g.Y = gp(p.h); g.ldy = p.H; g.ssq_out = gp(p.ssq); g.ssq_ld = p.ssq_ld;
          g.part = gp(p.dpart); g.ngroups = p.d_groups;
          gemm_os_epilogue_body<DT, EPI_RESID, 2, STEP_DNT, true>(g, p.d_splits, dgrp, 0, tid);
        }
      }
      if (l + 1 < L) {
        bar_arrive(sync_of(p.sync), nbar + 1);
        if (b < p.nt_q) q_issue(l + 1);
        if (!bar_wait(sync_of(p.sync), ++nbar, &flag_s)) return;
      }
    }
  }
  if (threadIdx.x == 0) {
    wait_memory();
    trace_at(sync_of(pp->sync), 0, 1);
  }
}

}  // namespace fdllm
