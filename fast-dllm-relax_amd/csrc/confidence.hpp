// Per-row confidence from the lm_head's 256-column tile statistics, and the threshold unmask rule.
//
// confidence_row: one wave combines a row's tiles into (first argmax, maxp = 1 / sum exp(logit - max))
// in the fixed lane order oracle/confidence.c defines (fd_combine), so that the two agree bit for bit
// (the device restatement of shifted_confidence / get_confidence_m*, fast_dllm_relax/runtime.py:158-181,
// model/metal.py:316-374).
//
// unmask_wave: the threshold rule of the decode loop (runtime.py:794-805) on one sub-block, with the
// shift of runtime.py:172-174 (block row s0 + r takes the prediction of confidence row row0 + r - 1;
// confidence row 0 keeps its own): the masked rows whose probability is above the threshold are
// unmasked, and when there is none, the first masked row of largest probability.  Lane r < sub takes
// sub-block row r.
#pragma once
#include "common.hpp"
#include "kernels.hpp"

namespace fdllm {

__device__ __forceinline__ void confidence_row(const float* m, const int32_t* am, const float* s, int tiles, int lane,
                                               int32_t* id_out, float* p_out) {
#pragma clang fp contract(off)
  float vmax = -INFINITY;
  int amax = 0x7fffffff;
  for (int t = lane; t < tiles; t += 64) {
    const float x = m[t];
    if (x > vmax) { vmax = x; amax = am[t]; }
  }
  for (int k = 32; k >= 1; k >>= 1) {
    const float ov = __shfl_xor(vmax, k, WAVE);
    const int oa = __shfl_xor(amax, k, WAVE);
    if (ov > vmax || (ov == vmax && oa < amax)) { vmax = ov; amax = oa; }
  }
  float acc = 0.0f;
  for (int t = lane; t < tiles; t += 64) {
    const float wgt = s[t] * fd_exp_neg(m[t] - vmax);
    acc = acc + wgt;
  }
  for (int k = 32; k >= 1; k >>= 1) acc = acc + __shfl_xor(acc, k, WAVE);
  *id_out = amax;
  *p_out = 1.0f / acc;
}

// The same combine for NR rows at once, each row's statistics requested together before any is used
// (one memory round trip for all of them instead of two per row, one per loop above); rows past the
// last (nr) and tiles past `tiles` take no part.  tiles <= 64 NT.
template <int NR, int NT>
__device__ __forceinline__ void confidence_rows(const float* m, const int32_t* am, const float* s, int tiles,
                                                int stride, int nr, int lane, int32_t* id_out, float* p_out) {
#pragma clang fp contract(off)
  float mv[NR][NT], sv[NR][NT];
  int32_t av[NR][NT];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      const int t = lane + 64 * i;
      const bool ok = r < nr && t < tiles;
      const size_t o = (size_t)r * stride + t;
      mv[r][i] = ok ? m[o] : -INFINITY;
      av[r][i] = ok ? am[o] : 0x7fffffff;
      sv[r][i] = ok ? s[o] : 0.f;
    }
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    float vmax = -INFINITY;
    int amax = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < NT; ++i)
      if (lane + 64 * i < tiles && mv[r][i] > vmax) { vmax = mv[r][i]; amax = av[r][i]; }
    for (int k = 32; k >= 1; k >>= 1) {
      const float ov = __shfl_xor(vmax, k, WAVE);
      const int oa = __shfl_xor(amax, k, WAVE);
      if (ov > vmax || (ov == vmax && oa < amax)) { vmax = ov; amax = oa; }
    }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NT; ++i)
      if (lane + 64 * i < tiles) {
        const float wgt = sv[r][i] * fd_exp_neg(mv[r][i] - vmax);
        acc = acc + wgt;
      }
    for (int k = 32; k >= 1; k >>= 1) acc = acc + __shfl_xor(acc, k, WAVE);
    id_out[r] = amax;
    p_out[r] = 1.0f / acc;
  }
}

// ids / maxp: the call's unshifted confidence (any memory the wave can read).  One wave; the block is
// at most 64 rows (lane j holds block row j) and lanes < sub take the sub-block rows.
__device__ __forceinline__ void unmask_wave(const int32_t* ids, const float* maxp, const UnmaskP& u, int lane) {
  const int32_t old = lane < u.bd ? u.block[lane] : 0;
  const int32_t mine = __shfl(old, min(u.s0 + lane, 63), WAVE);  // block row s0 + lane
  int32_t id = 0;
  float p = 0.f;
  bool masked = false;
  if (lane < u.sub) {
    const int i = u.row0 + lane;
    const int src = i > 0 ? i - 1 : 0;
    id = ids[src];
    p = maxp[src];
    masked = mine == u.mask_id;
  }
  const unsigned long long mm = __ballot(masked);
  bool sel = masked && p > u.thr;
  unsigned long long sm = __ballot(sel);
  if (sm == 0ull && mm != 0ull) {
    // top-1 fallback: the first masked row of largest probability
    float bp = masked ? p : -INFINITY;
    int br = masked ? lane : 64;
    for (int k = 32; k >= 1; k >>= 1) {
      const float op = __shfl_xor(bp, k, WAVE);
      const int orr = __shfl_xor(br, k, WAVE);
      if (op > bp || (op == bp && orr < br)) { bp = op; br = orr; }
    }
    sel = lane == br;
    sm = __ballot(sel);
  }
  if (sel) u.block[u.s0 + lane] = id;
  if (u.report == nullptr) return;
  // the block after the update, from registers: row j = s0 + r takes lane r's result
  const int32_t upd = sel ? id : mine;
  const int r = lane - u.s0;
  const int32_t moved = __shfl(upd, r >= 0 && r < u.sub ? r : 0, WAVE);
  int32_t* rep = u.report;
  if (lane < u.bd) rep[REP_BLOCK + lane] = r >= 0 && r < u.sub ? moved : old;
  if (lane < u.sub) {
    rep[REP_BLOCK + u.bd + lane] = id;
    rep[REP_BLOCK + u.bd + u.sub + lane] = __float_as_int(p);
  }
  if (lane == 0) {
    rep[REP_LEFT] = __popcll(mm & ~sm);
    rep[REP_COUNT] = __popcll(sm);
    rep[REP_LAST] = ids[u.rows - 1];
    // the 64-bit row masks as (low, high) word pairs: sub-blocks of up to 64 rows
    rep[REP_BLOCK + u.bd + 2 * u.sub] = (int32_t)(unsigned)mm;
    rep[REP_BLOCK + u.bd + 2 * u.sub + 1] = (int32_t)(unsigned)(mm >> 32);
    rep[REP_BLOCK + u.bd + 2 * u.sub + 2] = (int32_t)(unsigned)sm;
    rep[REP_BLOCK + u.bd + 2 * u.sub + 3] = (int32_t)(unsigned)(sm >> 32);
  }
  // the report may be host memory the caller polls: every lane's stores reach it before lane 0
  // publishes the sequence number
  __threadfence_system();
  __builtin_amdgcn_wave_barrier();
  if (lane == 0) __hip_atomic_store(rep + REP_SEQ, u.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace fdllm
