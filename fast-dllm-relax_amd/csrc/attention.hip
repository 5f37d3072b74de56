// Attention launch planning and launchers; the kernels and their bodies are in attn_body.hpp.
#include "attn_body.hpp"

#include <algorithm>

namespace fdllm {

// The chunked kernel's workgroup: query tiles x 2 key parts, 2 query tiles for one sequence and 4 for a
// batched call.  A query's arithmetic does not depend on how many tiles share its workgroup, so the
// results are those of the 4-tile workgroups; with twice the workgroups more compute units take each
// chunk's keys (one sequence, 1.5B, prefix 2048, chunk + merge per layer: 13.0 -> 12.3 us at 32 rows).
// The chunk length is chosen on the 4-tile count for both, so that it, and with it every result, stays
// the same.  (4 key parts of 32 keys measured faster still, 11.9 us, but a key part's online softmax
// then runs over other blocks, which changes the rounding; batched calls on 2 tiles: 128-row partial
// step 2.73 against 2.54 ms.)

// Launch plan: short row blocks (the cached decode step) use attn_chunk_kernel with one key chunk of
// CH keys per workgroup; long row blocks (prefill, stateless forward) use attn_kernel with few, long
// key ranges per workgroup.
AttnPlan attn_plan(int rows, int nq, int nkv, int Lk, int target_wgs, int nseq) {
  AttnPlan p{};
  const int QT = ((nq / nkv) * rows + 15) / 16;
  // chunked: 128 keys per workgroup unless that leaves fewer workgroups than aimed for; at most 64
  // chunks, so the split merge stays small (longer contexts take the loop kernel)
  if (QT <= 12 && (Lk + 127) / 128 <= 64) {
    p.chunked = 1;
    p.key_groups = 2;
    p.chunk = 128;
    if ((QT + 3) / 4 * nkv * ((Lk + 127) / 128) < target_wgs && (Lk + 63) / 64 <= 64) p.chunk = 64;
    p.q_tiles_per_wg = nseq > 1 ? 4 : 2;
    p.qg = (QT + p.q_tiles_per_wg - 1) / p.q_tiles_per_wg;
    p.S = (Lk + p.chunk - 1) / p.chunk;
    return p;
  }
  p.chunked = 0;
  if (QT >= 32) { p.q_tiles_per_wg = 4; p.key_groups = 1; }
  else { p.q_tiles_per_wg = 4; p.key_groups = 2; }
  p.qg = (QT + p.q_tiles_per_wg - 1) / p.q_tiles_per_wg;
  const int base = p.qg * nkv;
  const int max_splits = std::max(1, (Lk + 32 * p.key_groups - 1) / (32 * p.key_groups));
  int S = std::min(max_splits, std::max(1, (target_wgs + base - 1) / base));
  p.chunk = (((Lk + S - 1) / S) + 31) / 32 * 32;
  p.S = (Lk + p.chunk - 1) / p.chunk;
  return p;
}

size_t attn_partial_floats(const AttnP& a) {
  const int QT = ((a.nq / a.nkv) * a.rows + 15) / 16;
  return (size_t)std::max(a.nseq, 1) * a.nkv * QT * a.S * PSZ;
}

// the merge kernel whose register path covers S splits in one round trip where it can
template <int DT>
static auto merge_kernel_for(int S) {
  return S > 24 ? attn_merge_kernel<DT, 40> : attn_merge_kernel<DT, 24>;
}

template <typename K>
static void raise_lds(K kern, size_t lds) {
  // a runtime that needs no attribute for LDS up to the device limit may reject it: clear that error
  // and let the launch report whether the size fits
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
          hipSuccess)
    (void)hipGetLastError();
}

template <int DT, int QPW, int KSW>
static hipError_t launch_loop(const AttnP& a, const AttnPlan& p, hipStream_t st) {
  const size_t loop_lds = (size_t)KSW * (KB * KLD + HD * VLD) * 2;
  const size_t merge_lds = (size_t)2 * KSW * QPW * 16 * 4 + (size_t)(KSW - 1) * QPW * (HD / 16) * 64 * 16;
  const size_t lds = std::max(loop_lds, merge_lds);
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  auto kern = attn_kernel<DT, QPW, KSW>;
  raise_lds(kern, lds);
  hipLaunchKernelGGL(kern, dim3(p.qg, a.nkv, a.S), dim3(64 * QPW * KSW), lds, st, a);
  if (a.S > 1) {
    const int QT = ((a.nq / a.nkv) * a.rows + 15) / 16;
    hipLaunchKernelGGL(merge_kernel_for<DT>(a.S), dim3(HD / 16, QT, a.nkv), dim3(64), 0, st, a);
  }
  return hipGetLastError();
}

template <int DT, int CH, int KH, int MASK, int QPW>
static hipError_t launch_chunk_kh(const AttnP& a, const AttnPlan& p, hipStream_t st) {
  // K and V^T of the chunk, then (one-sequence calls) the queries the first key part shares
  const size_t loop_lds = (size_t)CH * KLD * 2 + (size_t)HD * (CH + 8) * 2 +
                          (KH > 1 && a.nseq <= 1 ? (size_t)QPW * 4 * 64 * 16 : 0);
  const size_t merge_lds = (size_t)2 * KH * QPW * 16 * 4 + (size_t)(KH - 1) * QPW * (HD / 16) * 64 * 16;
  const size_t lds = std::max(loop_lds, merge_lds);
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  const int nseq = std::max(a.nseq, 1);
  auto kern = attn_chunk_kernel<DT, QPW, KH, CH, MASK>;
  raise_lds(kern, lds);
  if (nseq == 1)
    hipLaunchKernelGGL(kern, dim3(attn_chunk_grid_1seq(p.qg, a.nkv, a.S)), dim3(64 * QPW * KH), lds, st, a);
  else
    hipLaunchKernelGGL(kern, dim3(p.qg * nseq, a.nkv, a.S), dim3(64 * QPW * KH), lds, st, a);
  if (a.S > 1) {
    const int QT = ((a.nq / a.nkv) * a.rows + 15) / 16;
    hipLaunchKernelGGL(merge_kernel_for<DT>(a.S), dim3(HD / 16, QT, a.nkv * nseq), dim3(64), 0, st, a);
  }
  return hipGetLastError();
}

// attn_plan's workgroup shape: 2 (one sequence) or 4 (batched) query tiles x 2 key parts
template <int DT, int CH, int MASK>
static hipError_t launch_chunk_shape(const AttnP& a, const AttnPlan& p, hipStream_t st) {
  if (p.key_groups != 2) return hipErrorInvalidValue;
  if (p.q_tiles_per_wg == 2) return launch_chunk_kh<DT, CH, 2, MASK, 2>(a, p, st);
  if (p.q_tiles_per_wg == 4) return launch_chunk_kh<DT, CH, 2, MASK, 4>(a, p, st);
  return hipErrorInvalidValue;
}
template <int DT, int CH>
static hipError_t launch_chunk_mask(const AttnP& a, const AttnPlan& p, hipStream_t st) {
  switch (a.mask) {
    case 0: return launch_chunk_shape<DT, CH, 0>(a, p, st);
    case 1: return launch_chunk_shape<DT, CH, 1>(a, p, st);
    default: return launch_chunk_shape<DT, CH, 2>(a, p, st);
  }
}

// Long row blocks: RoPE + KV append pass, then the flash-style kernel.  Two query heads per workgroup,
// as four waves of one query tile each, once that still gives 1024 workgroups; else one head (more
// workgroups win over fewer K/V re-reads below about that many).  Measured at 2048 and 8192 rows
// against three heads as two waves of three tiles (one wave per SIMD either way): 38.7 against 41.4 ms
// for the 8192-row prefill.  Three and six heads stay available through FDLLM_PREFILL_HPW.
template <int DT, int MASK, int TQ, int NWQ>
static hipError_t launch_prefill_cfg(const AttnP& a, int hpw, hipStream_t st) {
  constexpr size_t lds = 2 * ((size_t)64 * (HD + 8) + (size_t)HD * (64 + 8)) * 2;
  auto kern = attn_prefill_kernel<DT, MASK, TQ, NWQ>;
  raise_lds(kern, lds);
  const int nqb = (a.rows + 31) / 32, grp = a.nq / a.nkv;
  hipLaunchKernelGGL(kern, dim3(nqb * (grp / hpw), a.nkv), dim3(64 * NWQ), lds, st, a, hpw);
  return hipGetLastError();
}

// The paired-query-block kernel for models with 6 query heads per kv head: all heads of a kv head per
// workgroup (PAIR_TQ tiles per wave) from PAIR_WHOLE_MIN workgroups, below that the heads split over
// three workgroups (one tile per wave) from PAIR_SPLIT_MIN_BLOCKS query blocks, below that
// attn_prefill_kernel; and its K/V blocks in flight.  Measured (1.5B bf16 build_prefix_cache, ms; the
// one-block kernel / split / whole): 512 rows 3.31 / 3.38 / 3.82, 1024 4.95 / 4.89 / 5.58, 2048 8.44 /
// 8.03 / 9.12, 4096 16.68 / 15.93 / 15.58, 8192 34.2 / 34.3 / 29.4.
constexpr int PAIR_TQ = 3, PAIR_DEPTH = 3;
constexpr int PAIR_WHOLE_MIN = 128, PAIR_SPLIT_MIN_BLOCKS = 32;

template <int DT, int MASK, int TQ>
static hipError_t launch_pair(const AttnP& a, int pairs, int groups, hipStream_t st) {
  auto kern = attn_prefill_pair_kernel<DT, MASK, TQ, PAIR_DEPTH>;
  constexpr size_t lds = (size_t)(PAIR_DEPTH + 1) * 2 * 64 * HD * 2;  // K and V of D + 1 key blocks
  raise_lds(kern, lds);
  hipLaunchKernelGGL(kern, dim3(pairs, a.nkv, groups), dim3(256), lds, st, a);
  return hipGetLastError();
}

template <int DT, int MASK>
static hipError_t launch_prefill(const AttnP& a, hipStream_t st) {
  if (!a.roped) hipLaunchKernelGGL(rope_kv_kernel<DT>, dim3(a.rows), dim3(128), 0, st, a);
  const int nqb = (a.rows + 31) / 32, grp = a.nq / a.nkv;
  const int pairs = (nqb + 1) / 2;
  if (grp == 2 * PAIR_TQ) {
    // prefill_pair: 0 off, 1 by size, 2 always all heads per workgroup, 3 always the split form
    const bool whole = a.prefill_pair == 2 || (a.prefill_pair == 1 && pairs * a.nkv >= PAIR_WHOLE_MIN);
    const bool split = a.prefill_pair == 3 || (a.prefill_pair == 1 && !whole && nqb >= PAIR_SPLIT_MIN_BLOCKS);
    if (whole) return launch_pair<DT, MASK, PAIR_TQ>(a, pairs, 1, st);
    if (split) return launch_pair<DT, MASK, 1>(a, pairs, PAIR_TQ, st);
  }
  int hpw = grp % 2 == 0 && nqb * (grp / 2) * a.nkv >= 1024 ? 2 : 1;
  const int ph = a.prefill_hpw;
  if ((ph == 1 || ph == 2 || ph == 3 || ph == 6) && grp % ph == 0) hpw = ph;
  switch (hpw) {
    case 6: return launch_prefill_cfg<DT, MASK, 3, 4>(a, 6, st);
    case 3: return launch_prefill_cfg<DT, MASK, 3, 2>(a, 3, st);
    case 2: return launch_prefill_cfg<DT, MASK, 1, 4>(a, 2, st);
    default: return launch_prefill_cfg<DT, MASK, 1, 2>(a, 1, st);
  }
}

// the prefill kernel takes row blocks of at least this many rows without an explicit bias
constexpr int PREFILL_MIN_ROWS = 128;

// Batched calls without a mask: the RoPE + KV append pass over the call's rows, then attn_seq_kernel with
// its key blocks SEQ_DEPTH ahead and SEQ_KH key parts (waves per query tile).
constexpr int SEQ_DEPTH = 3;
#ifndef FD_SEQ_KH
#define FD_SEQ_KH 2
#endif
#ifndef FD_SEQ_NQW
#define FD_SEQ_NQW 2
#endif
constexpr int SEQ_KH = FD_SEQ_KH, SEQ_NQW = FD_SEQ_NQW;

size_t plan_seq_units(AttnP& a, int ncu) {
  const int QT = ((a.nq / a.nkv) * a.rows + 15) / 16, xg = (QT + SEQ_NQW - 1) / SEQ_NQW;
  int T[MAX_SEQS], s[MAX_SEQS];
  for (int b = 0; b < a.nseq; ++b) {
    T[b] = std::max(1, (a.seq_lk[b] + 63) / 64);
    s[b] = 1;
  }
  int units = a.nseq;
  const bool cnt_ok = a.seq_cnt != nullptr && (size_t)a.nseq * a.nkv * xg * SEQ_NQW <= (size_t)SEQ_CNT_MAX;
  const int cap = cnt_ok && ncu > 0 ? std::min(MAX_SEQ_UNITS, std::max(a.nseq, ncu / (a.nkv * xg))) : a.nseq;
  while (units < cap) {
    int best = 0, bl = 0;
    for (int b = 0; b < a.nseq; ++b) {
      const int l = (T[b] + s[b] - 1) / s[b];
      if (l > bl) { bl = l; best = b; }
    }
    if (bl <= 2 || s[best] >= 16) break;
    ++s[best];
    ++units;
  }
  // sequence-major units (u0 + j indexes the partials), launched longest first: units past what one
  // round of workgroups holds wait for the first to finish, and the shortest wait at least cost
  int ua[MAX_SEQ_UNITS], ut[MAX_SEQ_UNITS], ord[MAX_SEQ_UNITS];
  int u = 0;
  for (int b = 0; b < a.nseq; ++b)
    for (int j = 0; j < s[b]; ++j, ++u) {
      ua[u] = b | (j << 6) | (s[b] << 11) | ((u - j) << 16);
      ut[u] = (T[b] * j / s[b]) | ((T[b] * (j + 1) / s[b]) << 16);
      ord[u] = u;
    }
  auto len = [&](int v) { return (ut[v] >> 16) - (ut[v] & 0xffff); };
  std::stable_sort(ord, ord + u, [&](int x, int y) { return len(x) > len(y); });
  for (int v = 0; v < u; ++v) {
    a.unit_a[v] = ua[ord[v]];
    a.unit_t[v] = ut[ord[v]];
  }
  a.nunits = u;
  return units > a.nseq ? (size_t)u * a.nkv * xg * SEQ_NQW * PSZ : 0;
}

template <int DT>
static hipError_t launch_seq(const AttnP& a, hipStream_t st) {
  if (a.nunits < a.nseq || a.nunits > MAX_SEQ_UNITS) return hipErrorInvalidValue;
  if (!a.roped) hipLaunchKernelGGL(rope_kv_kernel<DT>, dim3(a.nseq * a.rows), dim3(128), 0, st, a);
  const int QT = ((a.nq / a.nkv) * a.rows + 15) / 16, xg = (QT + SEQ_NQW - 1) / SEQ_NQW;
  const int pairs = a.nunits * a.nkv;
  auto kern = attn_seq_kernel<DT, SEQ_DEPTH, SEQ_NQW, SEQ_KH>;
  constexpr size_t lds = (size_t)(SEQ_DEPTH + 1) * 2 * 64 * HD * 2;  // K and V of D + 1 key blocks
  raise_lds(kern, lds);
  hipLaunchKernelGGL(kern, dim3((pairs + 7) / 8 * 8 * xg), dim3(64 * SEQ_NQW * SEQ_KH), lds, st, a);
  return hipGetLastError();
}

bool attn_takes_roped(const AttnP& a) {
  if (a.nseq > 1 && a.seq_attn && a.mask == 0) return true;
  const AttnPlan p = attn_plan(a.rows, a.nq, a.nkv, a.Lk, a.target_wgs, a.nseq);
  return !p.chunked && a.nseq <= 1 && a.rows >= PREFILL_MIN_ROWS && a.mask != 2;
}

template <int DT>
static hipError_t launch_dt(const AttnP& a, hipStream_t st) {
  const AttnPlan p = attn_plan(a.rows, a.nq, a.nkv, a.Lk, a.target_wgs, a.nseq);
  if (a.roped && !attn_takes_roped(a)) return hipErrorInvalidValue;
  if (p.S != a.S || p.chunk != a.chunk) return hipErrorInvalidValue;
  if (a.ofrag && (a.nseq > 1 || a.rows > 32)) return hipErrorInvalidValue;
  if (a.nseq > MAX_SEQS) return hipErrorInvalidValue;
  if (a.nseq > 1 && a.seq_attn && a.mask == 0) return launch_seq<DT>(a, st);
  if (a.nseq > 1 && !p.chunked) return hipErrorInvalidValue;
  if (!p.chunked && a.nseq <= 1 && a.rows >= PREFILL_MIN_ROWS && a.mask != 2) {
    if (a.mask == 1) return launch_prefill<DT, 1>(a, st);
    return launch_prefill<DT, 0>(a, st);
  }
  if (p.chunked) {
    if (p.chunk == 128) return launch_chunk_mask<DT, 128>(a, p, st);
    return launch_chunk_mask<DT, 64>(a, p, st);
  }
  if (p.key_groups == 1) return launch_loop<DT, 4, 1>(a, p, st);
  return launch_loop<DT, 4, 2>(a, p, st);
}

hipError_t launch_attention(int dt, const AttnP& a, hipStream_t st) {
  if (dt == DT_BF16) return launch_dt<DT_BF16>(a, st);
  return launch_dt<DT_F16>(a, st);
}

}  // namespace fdllm
