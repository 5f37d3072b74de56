// Skinny projection GEMMs of the cached step over packed weights: Y[M, N] = X[M, K] . W[N, K]^T with
// M <= 32 rows per m-chunk (gridDim.z), fp32 accumulation on MFMA 16x16x32.
//
// Work split.  A workgroup owns TW x TPW consecutive 16-row weight tiles and the k steps of one
// cross-workgroup split (gridDim.y).  Its TW x KW waves are arranged as TW tile columns times KW k
// partitions: wave (tw, kw) streams its TPW tiles' packed 1 KB blocks for its share of the k steps,
// U steps per load group, double-buffered, and multiplies them with the matching activation
// fragments (B operand, read from the row-major activations and transformed on the fly).  The KW
// partial sums are added in LDS in fixed order; gridDim.y > 1 splits are added by the workgroup that
// arrives last, in split order, so every result is deterministic.
//
// Epilogues follow the reference's rounding points (fast_dllm_relax/model/cuda.py):
//   EPI_BIAS       y = rnd(acc + b[n])                              qkv_proj + bias (cuda.py:389-399)
//   EPI_RESID      h = rnd(h + rnd(acc)), plus row sums of squares  o_proj / down_proj + residual
//                  of the new h per 16-column tile for the next RMSNorm   (cuda.py:561-579)
//   EPI_SILU_PAIR  act = rnd(rnd(silu(rnd(g))) * rnd(u))             gate_up + _silu_fp32 * up (cuda.py:319-348)
//   EPI_LOGITS     logits fp32 = rnd(acc) and per-256-column confidence statistics (cuda.py:704-711)
// XF_RMS applies FastDLLMRMSNorm (cuda.py:269-275) to the activations as they are loaded:
//   x' = rnd(w[k] * rnd(x * inv_rms[m])), inv_rms from the sums of squares the producer left.
#pragma once
#include "common.hpp"
#include "kernels.hpp"

namespace fdllm {

#ifdef FD_WLOAD_PLAIN
#define FD_WLOAD(p) (*(p))
#else
#define FD_WLOAD(p) __builtin_nontemporal_load(p)
#endif

__device__ __forceinline__ const u32x4* wblock(const u16* W, int KS, int t, int s) {
  return reinterpret_cast<const u32x4*>(W + ((size_t)t * KS + s) * 512) + (threadIdx.x & 63);
}

// A k split's fp32 sums of one (16-column tile t, 16-row block b) unit, lane (lr, lg) holding rows
// 16 b + lr, columns 16 t + 4 lg .. + 3: in the unit layout the split-sum kernel reads
// (part[split][tile][block][lane]), or with a.part_rows row-major (part[split][M][N]) for a caller that
// sums the splits itself.
__device__ __forceinline__ void store_split_unit(const GemmP& a, int split, int t, int b, int lane, const f32x4& v) {
  const int nblk = (a.M + 15) / 16;
  if (t >= a.ntiles || b >= nblk) return;
  if (a.part_rows) {
    const int m = 16 * b + (lane & 15), n = 16 * t + 4 * (lane >> 4);
    if (m < a.M && n < a.N) *reinterpret_cast<f32x4*>(a.part + ((size_t)split * a.M + m) * a.N + n) = v;
  } else {
    reinterpret_cast<f32x4*>(a.part)[(((size_t)split * a.ntiles + t) * nblk + b) * 64 + lane] = v;
  }
}

template <int DT, int XF>
__device__ __forceinline__ u32x4 xform(u32x4 raw, u32x4 wv, float inv) {
  if constexpr (XF == XF_NONE) {
    return raw;
  } else if constexpr (DT == DT_BF16) {
    // the same two roundings per value as below, each pair rounded by one packed conversion and the
    // products unpacked by a shift and a mask (the per-value form took 15 instructions per pair, this
    // one 10: one-shot qkv and gate_up transform every activation of the call in each workgroup)
    u32x4 o;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t r = pack_f32x2<DT>(__uint_as_float(raw[c] << 16) * inv, __uint_as_float(raw[c] & 0xffff0000u) * inv);
      o[c] = pack_f32x2<DT>(__uint_as_float(wv[c] << 16) * __uint_as_float(r << 16),
                            __uint_as_float(wv[c] & 0xffff0000u) * __uint_as_float(r & 0xffff0000u));
    }
    return o;
  } else {
    u32x4 o;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float y0 = lo_f32<DT>(wv[c]) * rnd<DT>(lo_f32<DT>(raw[c]) * inv);
      float y1 = hi_f32<DT>(wv[c]) * rnd<DT>(hi_f32<DT>(raw[c]) * inv);
      o[c] = pack2(from_f32<DT>(y0), from_f32<DT>(y1));
    }
    return o;
  }
}

// Confidence statistics of one block's 256-column logit tile, held in LDS as [BM][256] values (model
// dtype, or fp32 already rounded to it): one wave per row (rows w, w + NW, ...) reduces the row's columns to (max, first argmax, sum of
// exp(x - max)) with one lane order and reduction order, so every kernel that produces the tile gives
// identical bits.  A wave works on RP of its rows at once, and the cross-lane steps are
// register exchanges (lane_down) instead of LDS permutes: each row's reduction is a chain of exchanges
// whose latency, one row at a time through LDS, cost more than the tile's MFMAs.
template <int DT> __device__ __forceinline__ float tile_value(u16 v) { return to_f32<DT>(v); }
template <int DT> __device__ __forceinline__ float tile_value(float v) { return v; }

template <int DT, int BM, int NW, typename T>
__device__ __forceinline__ void logits_tile_stats(const GemmP& a, const T* tile, int m0, int nb, int w, int lane) {
  constexpr int RPW = BM / NW;  // rows of each wave
  constexpr int RP = RPW % 4 == 0 ? 4 : (RPW % 2 == 0 ? 2 : 1);
  static_assert(BM % NW == 0, "whole rows per wave");
  const int n0 = nb * 256;
  const bool whole = n0 + 256 <= a.N;  // every column of the tile is a vocabulary entry
  for (int ml0 = w; ml0 < BM; ml0 += NW * RP) {
    if (m0 + ml0 >= a.M) break;
    float x[RP][4], vmax[RP];
    int amax[RP];
    // the row max (NaN never wins): per lane over its columns, then a shift-down tree into lane 0
#pragma unroll
    for (int r = 0; r < RP; ++r) {
      const T* row = tile + (ml0 + NW * r) * 256;
      vmax[r] = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = lane + 64 * i;
        x[r][i] = tile_value<DT>(row[c]);
        if ((whole || n0 + c < a.N) && x[r][i] > vmax[r]) vmax[r] = x[r][i];
      }
    }
    static_for<0, 6>([&](auto s) {
      constexpr int k = 32 >> decltype(s)::value;
#pragma unroll
      for (int r = 0; r < RP; ++r) {
        const float o = lane_down<k>(vmax[r]);
        vmax[r] = o > vmax[r] ? o : vmax[r];
      }
    });
    // the first column holding it (none when the max is -inf): the smallest candidate index, by a min tree
#pragma unroll
    for (int r = 0; r < RP; ++r) {
      vmax[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vmax[r]), 0));
      amax[r] = 0x7fffffff;
#pragma unroll
      for (int i = 3; i >= 0; --i) {
        const int c = lane + 64 * i;
        if ((whole || n0 + c < a.N) && x[r][i] == vmax[r] && vmax[r] > -INFINITY) amax[r] = n0 + c;
      }
    }
    static_for<0, 6>([&](auto s) {
      constexpr int k = 32 >> decltype(s)::value;
#pragma unroll
      for (int r = 0; r < RP; ++r) amax[r] = min(amax[r], lane_down<k>(amax[r]));
    });
    float sum[RP];
    {
#pragma clang fp contract(off)
#pragma unroll
      for (int r = 0; r < RP; ++r) {
        sum[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (whole || n0 + lane + 64 * i < a.N) sum[r] = sum[r] + fd_exp_neg(x[r][i] - vmax[r]);
      }
      // the butterfly's sum order, in lane 0
      static_for<0, 6>([&](auto s) {
        constexpr int k = 32 >> decltype(s)::value;
#pragma unroll
        for (int r = 0; r < RP; ++r) sum[r] = sum[r] + lane_down<k>(sum[r]);
      });
    }
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < RP; ++r) {
        if (m0 + ml0 + NW * r >= a.M) break;
        const size_t o = (size_t)(m0 + ml0 + NW * r) * a.stat_tiles + nb;
        a.stat_m[o] = vmax[r];
        a.stat_a[o] = amax[r];
        a.stat_s[o] = sum[r];
      }
    }
  }
}

template <int DT, int EPI, int XF, int MT, int TPW, int TW, int KW, int U>
__global__ __launch_bounds__(64 * TW * KW) void gemm_pk_kernel(GemmP a) {
  __shared__ float inv_s[32];
  __shared__ int flag_s;
  extern __shared__ __align__(16) unsigned char smem[];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int tw = w % TW, kw = w / TW;
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = blockIdx.z * 32;
  // the workgroup's column group bx and k split by of ny: (blockIdx.x, blockIdx.y) of gridDim.y, except in
  // a tail split, where workgroups tail_full + j take column group tail_full + j / tail_split, split
  // j % tail_split of the k steps
  int bx = blockIdx.x, by = blockIdx.y, ny = gridDim.y, kps = a.kps;
  if (a.tail_split > 1 && bx >= a.tail_full) {
    const int j = bx - a.tail_full;
    bx = a.tail_full + j / a.tail_split;
    by = j % a.tail_split;
    ny = a.tail_split;
    kps = a.KS / a.tail_split;
    // its compute unit also runs two whole groups: ahead of them in issue, a split finishes its third of
    // the k steps early and its hand-off and epilogue run while they stream, off the launch's critical
    // path (at equal priority all three finish together and the last arriver's hand-off comes last)
    __builtin_amdgcn_s_setprio(2);
  }
  const int t0 = (bx * TW + tw) * TPW;
  const int kq = kps / KW, kr = kps % KW;
  const int wb = by * kps + kw * kq + min(kw, kr);
  const int wn = kq + (kw < kr ? 1 : 0);

  // Every load below is unconditional and in bounds, so the compiler can count outstanding loads
  // exactly and keep the next group in flight while this one is multiplied: rows past M read row M - 1
  // (their products land in output rows that are discarded) and the prefetch past the last group
  // re-reads the last group.
  const int ngf = wn / U;  // full groups of U k steps; the rest run one step at a time
  const int mlast = a.M - 1;
  // a group's operands: weight blocks A, activation fragments X and (XF_RMS) the norm weights N
  constexpr int UN = XF == XF_RMS ? U : 1;
  u32x4 A0[U][TPW], A1[U][TPW], X0[U][MT], X1[U][MT], N0[UN], N1[UN];
  auto load = [&](int g, u32x4(&A)[U][TPW], u32x4(&X)[U][MT], u32x4(&Nw)[UN]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = wb + g * U + u;
#pragma unroll
      for (int j = 0; j < TPW; ++j) A[u][j] = __builtin_nontemporal_load(wblock(a.W, a.KS, t0 + j, s));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = min(m0 + 16 * mt + lr, mlast);
        X[u][mt] = *reinterpret_cast<const u32x4*>(a.X + (size_t)m * a.ldx + 32 * s + 8 * lg);
      }
      if constexpr (XF == XF_RMS) Nw[u] = *reinterpret_cast<const u32x4*>(a.nw + 32 * s + 8 * lg);
    }
  };
  if (ngf > 0) load(0, A0, X0, N0);

  float inv[MT];
  if constexpr (XF == XF_RMS) {
    // inv_rms of the chunk's 32 rows: 8 threads per row each add every 8th tile's sum of squares (all
    // loads in flight at once), then a fixed-order butterfly over the 8
    static_assert(64 * TW * KW >= 256, "the RMS prologue needs 256 threads");
    if (threadIdx.x < 256) {
      const int mr = threadIdx.x >> 3, pp = threadIdx.x & 7;
      const int m = m0 + mr;
      float v[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int t = pp + 8 * q;
        v[q] = (m < a.M && t < a.ssq_tiles) ? a.ssq[(size_t)t * a.ssq_ld + m] : 0.f;
      }
      float ss = 0.f;
#pragma unroll
      for (int q = 0; q < 16; ++q) ss += v[q];
      for (int q = 16; pp + 8 * q < a.ssq_tiles; ++q) ss += (m < a.M) ? a.ssq[(size_t)(pp + 8 * q) * a.ssq_ld + m] : 0.f;
      ss += __shfl_xor(ss, 1, WAVE);
      ss += __shfl_xor(ss, 2, WAVE);
      ss += __shfl_xor(ss, 4, WAVE);
      if (pp == 0) inv_s[mr] = 1.0f / sqrtf(ss / (float)a.H + a.eps);
    }
    __syncthreads();
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) inv[mt] = inv_s[16 * mt + lr];
  } else {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) inv[mt] = 1.f;
  }

  f32x4 acc[TPW][MT];
#pragma unroll
  for (int j = 0; j < TPW; ++j)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[j][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto comp = [&](u32x4(&A)[U][TPW], u32x4(&X)[U][MT], u32x4(&Nw)[UN]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      u32x4 b[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) b[mt] = xform<DT, XF>(X[u][mt], Nw[XF == XF_RMS ? u : 0], inv[mt]);
#pragma unroll
      for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[j][mt] = mfma16<DT>(A[u][j], b[mt], acc[j][mt]);
    }
  };
  // the scheduling barriers keep each prefetch ahead of the multiply it overlaps (the scheduler would
  // otherwise sink the loads below it and leave only one group in flight)
  for (int g = 0; g < ngf; g += 2) {
    load(min(g + 1, ngf - 1), A1, X1, N1);
    __builtin_amdgcn_sched_barrier(0);
    comp(A0, X0, N0);
    __builtin_amdgcn_sched_barrier(0);
    load(min(g + 2, ngf - 1), A0, X0, N0);
    __builtin_amdgcn_sched_barrier(0);
    if (g + 1 < ngf) comp(A1, X1, N1);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int s = wb + ngf * U; s < wb + wn; ++s) {  // remainder, one k step at a time
    u32x4 A[TPW], b[MT];
#pragma unroll
    for (int j = 0; j < TPW; ++j) A[j] = __builtin_nontemporal_load(wblock(a.W, a.KS, t0 + j, s));
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = min(m0 + 16 * mt + lr, mlast);
      const u32x4 wv = XF == XF_RMS ? *reinterpret_cast<const u32x4*>(a.nw + 32 * s + 8 * lg) : u32x4{0u, 0u, 0u, 0u};
      b[mt] = xform<DT, XF>(*reinterpret_cast<const u32x4*>(a.X + (size_t)m * a.ldx + 32 * s + 8 * lg), wv, inv[mt]);
    }
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[j][mt] = mfma16<DT>(A[j], b[mt], acc[j][mt]);
  }

  // ---- k partitions of the workgroup, added in LDS in fixed order ----
  if constexpr (KW > 1) {
    f32x4* red = reinterpret_cast<f32x4*>(smem);
    if (kw > 0) {
#pragma unroll
      for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) red[((((kw - 1) * TW + tw) * TPW + j) * MT + mt) * 64 + lane] = acc[j][mt];
    }
    __syncthreads();
    if (kw == 0) {
      for (int q = 1; q < KW; ++q)
#pragma unroll
        for (int j = 0; j < TPW; ++j)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[j][mt] += red[((((q - 1) * TW + tw) * TPW + j) * MT + mt) * 64 + lane];
    }
  }

  // ---- cross-workgroup k splits: the last arriver adds them in split order (its own from registers) ----
  if (ny > 1) {
    const size_t grp = (size_t)blockIdx.z * a.ngroups + bx;
    // the partials of the tail's groups only (tail_split: one row chunk), or of every group
    const size_t pgrp = a.tail_split > 1 ? (size_t)(bx - a.tail_full) : grp;
    constexpr unsigned per = TW * TPW * MT * 64;  // f32x4 per split partial
    const CohBuf pb = coh_buf(reinterpret_cast<f32x4*>(a.part) + pgrp * ny * per, (unsigned)ny * per * 16u);
    if (kw == 0) {
#pragma unroll
      for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          coh_stf4(pb, ((unsigned)by * per + ((tw * TPW + j) * MT + mt) * 64 + lane) * 16u, acc[j][mt]);
    }
    if (!arrive_last(a.counters + grp, ny, &flag_s)) return;
    if (kw == 0) {
      // every other split's partial is requested before any is added (one memory round trip per 16 splits)
      constexpr int SB = 16;
#pragma unroll
      for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const unsigned o = (((tw * TPW + j) * MT + mt) * 64 + lane) * 16u;
          f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
          for (int y0 = 0; y0 < ny; y0 += SB) {
            f32x4 v[SB];
#pragma unroll
            for (int q = 0; q < SB; ++q)
              v[q] = y0 + q < ny && y0 + q != by ? coh_ldf4(pb, (unsigned)(y0 + q) * per * 16u + o) : acc[j][mt];
#pragma unroll
            for (int q = 0; q < SB; ++q)
              if (y0 + q < ny) s = (y0 + q == 0) ? v[q] : s + v[q];
          }
          acc[j][mt] = s;
        }
    }
  }

  // ---- epilogues ----
  if constexpr (EPI == EPI_LOGITS) {
    // one workgroup = one 256-column confidence tile (TW * TPW == 16)
    float* tile = reinterpret_cast<float*>(smem);  // [32][256]
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + lr;
        const int nl = 16 * (tw * TPW + j) + 4 * lg;
        const int n = bx * 256 + nl;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = rnd<DT>(acc[j][mt][i]);
        *reinterpret_cast<f32x4*>(tile + m * 256 + nl) = f32x4{v[0], v[1], v[2], v[3]};
        if (a.logits != nullptr && m0 + m < a.M) {
          float* dst = a.logits + (size_t)(m0 + m) * a.ldl + n;
          if (n + 3 < a.N) {
            *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (n + i < a.N) dst[i] = v[i];
          }
        }
      }
    if (a.stat_m == nullptr) return;
    __syncthreads();
    logits_tile_stats<DT, 16 * MT, TW * KW>(a, tile, m0, bx, w, lane);
  } else if constexpr (EPI == EPI_SILU_PAIR) {
    if (kw != 0) return;
    const int p = t0 / 2;  // tiles t0 (gate) and t0 + 1 (up) of pair p
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = m0 + 16 * mt + lr;
      const int n = 16 * p + 4 * lg;
      if (m >= a.M || n >= a.N) continue;
      u16 out[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) out[i] = silu_mul<DT>(acc[0][mt][i], acc[1][mt][i]);
      *reinterpret_cast<u32x2*>(a.Y + (size_t)m * a.ldy + n) = u32x2{pack2(out[0], out[1]), pack2(out[2], out[3])};
    }
  } else {
    if (kw != 0) return;
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = m0 + 16 * mt + lr;
        const int n = 16 * (t0 + j) + 4 * lg;
        const bool ok = m < a.M && n < a.N;
        u16 out[4];
        float ss = 0.f;
        if (ok) {
          if constexpr (EPI == EPI_BIAS) {
#pragma unroll
            for (int i = 0; i < 4; ++i) out[i] = from_f32<DT>(acc[j][mt][i] + to_f32<DT>(a.bias[n + i]));
          } else {
            const u32x2 hv = *reinterpret_cast<const u32x2*>(a.Y + (size_t)m * a.ldy + n);
            const float hf[4] = {lo_f32<DT>(hv[0]), hi_f32<DT>(hv[0]), lo_f32<DT>(hv[1]), hi_f32<DT>(hv[1])};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              out[i] = from_f32<DT>(hf[i] + rnd<DT>(acc[j][mt][i]));
              const float y = to_f32<DT>(out[i]);
              ss += y * y;
            }
          }
          *reinterpret_cast<u32x2*>(a.Y + (size_t)m * a.ldy + n) = u32x2{pack2(out[0], out[1]), pack2(out[2], out[3])};
        }
        if constexpr (EPI == EPI_RESID) {
          ss += __shfl_xor(ss, 16, WAVE);
          ss += __shfl_xor(ss, 32, WAVE);
          if (lg == 0 && m < a.M && 16 * (t0 + j) < a.N) a.ssq_out[(size_t)(t0 + j) * a.ssq_ld + m] = ss;
        }
      }
  }
}

// Epilogue of one unit (a 16-row block of one tile, or of a gate/up tile pair): lane holds rows m
// (= m0 + 16 mt + lr) and columns 16 t + 4 lg .. + 3 of the sums v.
template <int DT, int EPI, int TPU, bool COH>
__device__ __forceinline__ void os_epilogue(const GemmP& a, const f32x4 (&v)[TPU], int m, int t, int lg) {
  if constexpr (EPI == EPI_SILU_PAIR) {
    const int n = 16 * (t / 2) + 4 * lg;
    if (m < a.M && n < a.N) {
      u16 out[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) out[i] = silu_mul<DT>(v[0][i], v[TPU - 1][i]);
      const size_t o = a.yfrag == 1 ? frag_off(m, n) : a.yfrag == 2 ? frag_blk_off(m, n, a.ldy >> 5) : (size_t)m * a.ldy + n;
      st8<COH>(a.Y + o, u32x2{pack2(out[0], out[1]), pack2(out[2], out[3])});
    }
  } else {
    const int n = 16 * t + 4 * lg;
    const bool ok = m < a.M && n < a.N;
    u16* y = a.Y + (EPI == EPI_RESID && a.yfrag ? frag_off(m, n) : (size_t)m * a.ldy + n);
    u16 out[4];
    float ss = 0.f;
    if (ok) {
      if constexpr (EPI == EPI_BIAS) {
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = from_f32<DT>(v[0][i] + to_f32<DT>(a.bias[n + i]));
      } else {
        const u32x2 hv = ld8<COH>(y);
        const float hf[4] = {lo_f32<DT>(hv[0]), hi_f32<DT>(hv[0]), lo_f32<DT>(hv[1]), hi_f32<DT>(hv[1])};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          out[i] = from_f32<DT>(hf[i] + rnd<DT>(v[0][i]));
          const float y = to_f32<DT>(out[i]);
          ss += y * y;
        }
      }
      st8<COH>(y, u32x2{pack2(out[0], out[1]), pack2(out[2], out[3])});
    }
    if constexpr (EPI == EPI_RESID) {
      ss += __shfl_xor(ss, 16, WAVE);
      ss += __shfl_xor(ss, 32, WAVE);
      if (lg == 0 && m < a.M && 16 * t < a.N) stf<COH>(a.ssq_out + (size_t)t * a.ssq_ld + m, ss);
    }
  }
}

// One-shot configurations of the four projections: tiles per workgroup, max k steps per wave, preferred
// k split (1.5B shapes: qkv 128 workgroups of 1 tile x 48 k steps, o_proj 96 of 1 x 48, gate_up 188 of
// 3 pairs x 48, down 24 x 10 of 4 tiles x 28).
constexpr int OsQkvNT = 1, OsQkvKPW = 6, OsQkvSplit = 1;
constexpr int OsOprojNT = 1, OsOprojKPW = 6, OsOprojSplit = 1;
constexpr int OsGateUpNT = 6, OsGateUpKPW = 6, OsGateUpSplit = 1;
constexpr int OsDownNT = 4, OsDownKPW = 5, OsDownSplit = 10;

// ---- one-shot skinny GEMM (M <= 32 rows per m-chunk) --------------------------------------------
// A workgroup of NW = 8 waves owns NT consecutive 16-row weight tiles and the k steps of one
// cross-workgroup split (gridDim.y).  Every wave requests all of its packed weight blocks at once (its
// share of the split's k steps for all NT tiles, at most KPW steps), so the workgroup's whole weight
// slice is in flight together.  The activation rows of the split are loaded once per workgroup,
// normalised (XF_RMS) and kept in LDS in MFMA fragment order.  The waves' partial sums are added in
// LDS in wave order, one (tile or pair, 16-row block) per wave; with k splits (gridDim.y > 1) the
// workgroups store their sums and gemm_os_epilogue_kernel, launched next, adds them in split order.
// Results are deterministic.
// Body of one workgroup (tile group bx, k split by of gy splits, m-chunk bz).  With COH its activation
// loads and its stores are agent-scope, for a launch in which other workgroups produce its inputs; the
// per-operator kernels below use plain accesses.
template <int DT, int EPI, int XF, int MT, int NT, int KPW, bool COH>
__device__ __forceinline__ void gemm_os_body(const GemmP& a, int bx, int by, int bz, int gy, unsigned char* smem) {
  constexpr int NW = 8;
  constexpr int UNITS = (EPI == EPI_SILU_PAIR ? NT / 2 : NT) * MT;
  static_assert(UNITS <= NW, "one epilogue unit per wave");
  __shared__ float inv_s[32];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = bz * 16 * MT, mlast = a.M - 1;  // m-chunks of 16 MT rows
  const int t0 = bx * NT;
  const int kb = by * a.kps;  // first k step of the split
  const int kq = a.kps / NW, kr = a.kps % NW;
  const int ws = kq * w + min(w, kr), wn = kq + (w < kr ? 1 : 0);  // this wave's k steps [ws, ws + wn)
  u32x4* xl = reinterpret_cast<u32x4*>(smem);                      // [kps][MT][64] fragments

  // 1. inputs of the activation staging first (their waits then do not cover the weight loads)
  float ssv[16];
  if constexpr (XF == XF_RMS) {
    if (threadIdx.x < 256) {
      const int m = m0 + (threadIdx.x >> 3), pp = threadIdx.x & 7;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int t = pp + 8 * q;
        ssv[q] = (m < a.M && t < a.ssq_tiles) ? ldf<COH>(a.ssq + (size_t)t * a.ssq_ld + m) : 0.f;
      }
    }
  }
  // the split's norm weights go to LDS behind the fragments (one 16-byte chunk per thread)
  u32x4* nwl = xl + (size_t)a.kps * MT * 64;  // [kps * 4] chunks of 8 weights
  u32x4 nwv = {0u, 0u, 0u, 0u};
  if constexpr (XF == XF_RMS) {
    if ((int)threadIdx.x < a.kps * 4) nwv = *reinterpret_cast<const u32x4*>(a.nw + 32 * kb + 8 * threadIdx.x);
  }
  // activation fragments per thread: F1 requested before the weights, the rest (F2) after them, so
  // that the registers of both are never live at once (kps * MT * 64 <= 512 * (F1 + F2))
  constexpr int F1 = 6, F2 = 6;
  const int nfrag = a.kps * MT * 64;
  auto xload = [&](int f) {
    f = min(f, nfrag - 1);
    const int sl = f / (MT * 64), rem = f - sl * (MT * 64), mt = rem >> 6, l = rem & 63;
    const int m = min(m0 + 16 * mt + (l & 15), mlast);
    const int k = 32 * (kb + sl) + 8 * (l >> 4);
    return ld16<COH>(a.X + (size_t)m * a.ldx + k);
  };
  u32x4 xv[F1];
#pragma unroll
  for (int i = 0; i < F1; ++i) xv[i] = xload(threadIdx.x + 512 * i);
  // 2. the weight slice: KPW k steps x NT tiles per wave, all requested now (steps past wn re-read
  //    the wave's first step and are not multiplied)
  u32x4 A[KPW][NT];
#pragma unroll
  for (int s = 0; s < KPW; ++s)
#pragma unroll
    for (int j = 0; j < NT; ++j)
      A[s][j] = FD_WLOAD(wblock(a.W, a.KS, t0 + j, kb + (s < wn ? ws + s : min(ws, a.kps - 1))));

  // 3. 1 / rms of the chunk's rows, then the normalised fragments into LDS
  if constexpr (XF == XF_RMS) {
    if (threadIdx.x < 256) {
      float ss = 0.f;
#pragma unroll
      for (int q = 0; q < 16; ++q) ss += ssv[q];
      const int m = m0 + (threadIdx.x >> 3), pp = threadIdx.x & 7;
      for (int q = 16; pp + 8 * q < a.ssq_tiles; ++q) ss += (m < a.M) ? ldf<COH>(a.ssq + (size_t)(pp + 8 * q) * a.ssq_ld + m) : 0.f;
      ss += __shfl_xor(ss, 1, WAVE);
      ss += __shfl_xor(ss, 2, WAVE);
      ss += __shfl_xor(ss, 4, WAVE);
      if (pp == 0) inv_s[threadIdx.x >> 3] = 1.0f / sqrtf(ss / (float)a.H + a.eps);
    }
    if ((int)threadIdx.x < a.kps * 4) nwl[threadIdx.x] = nwv;
    __syncthreads();
  }
  auto xstore = [&](int f, u32x4 x) {
    if (f < nfrag) {
      if constexpr (XF == XF_RMS) {
        const int sl = f / (MT * 64), rem = f - sl * (MT * 64), mt = rem >> 6, l = rem & 63;
        xl[f] = xform<DT, XF>(x, nwl[sl * 4 + (l >> 4)], inv_s[16 * mt + (l & 15)]);
      } else {
        xl[f] = x;
      }
    }
  };
#pragma unroll
  for (int i = 0; i < F1; ++i) xstore(threadIdx.x + 512 * i, xv[i]);
  if (nfrag > 512 * F1) {
    u32x4 xw[F2];
#pragma unroll
    for (int i = 0; i < F2; ++i) xw[i] = xload(threadIdx.x + 512 * (F1 + i));
#pragma unroll
    for (int i = 0; i < F2; ++i) xstore(threadIdx.x + 512 * (F1 + i), xw[i]);
  }
  __syncthreads();

  // 4. multiply: fragment (kstep s, block mt) read from LDS once per step for all NT tiles
  f32x4 acc[NT][MT];
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[j][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < KPW; ++s) {
    if (s < wn) {
      u32x4 b[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) b[mt] = xl[((ws + s) * MT + mt) * 64 + lane];
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[j][mt] = mfma16<DT>(A[s][j], b[mt], acc[j][mt]);
    }
  }

  // 5. the waves' partials into LDS (the activation region is free now), summed per unit in wave order
  __syncthreads();
  f32x4* red = reinterpret_cast<f32x4*>(smem);  // [NW][NT][MT][64]
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[((w * NT + j) * MT + mt) * 64 + lane] = acc[j][mt];
  __syncthreads();
  constexpr int TPU = EPI == EPI_SILU_PAIR ? 2 : 1;  // tiles per unit
  f32x4 v[TPU] = {};
  const int u = w;
  const bool has_unit = u < UNITS;
  const int ut = (u / MT) * TPU, umt = u % MT;  // unit's first tile (within the workgroup) and row block
  if (has_unit) {
#pragma unroll
    for (int q = 0; q < TPU; ++q) {
      f32x4 sum = red[((0 * NT + ut + q) * MT + umt) * 64 + lane];
      for (int ww = 1; ww < NW; ++ww) sum += red[((ww * NT + ut + q) * MT + umt) * 64 + lane];
      v[q] = sum;
    }
  }

  // 6. cross-workgroup k splits: the unit's partial, summed by the epilogue body
  if (gy > 1) {
    if (has_unit) {
      const size_t grp = (size_t)bz * a.ngroups + bx;
      constexpr int per = NT * MT * 64;  // f32x4 per split partial
      f32x4* part = reinterpret_cast<f32x4*>(a.part) + (grp * gy + by) * per;
#pragma unroll
      for (int q = 0; q < TPU; ++q) stf4<COH>(part + ((ut + q) * MT + umt) * 64 + lane, v[q]);
    }
    return;
  }
  if (has_unit) os_epilogue<DT, EPI, TPU, COH>(a, v, m0 + 16 * umt + lr, t0 + ut, lg);
}

// The same one-shot GEMM with the activations loaded straight into registers: a wave multiplies only
// its own k steps, so it loads only its own slice of the rows (MT 16-row blocks x its k steps, one
// 16-byte load per fragment), all at once and before its weight slice, and RMS-normalises them in
// registers.  Nothing goes through LDS but the norm weights, the 32 inverse RMS values and the wave
// sums, so the chain from launch to the first MFMA is one memory round trip.  Same k partition, same per-wave MFMA order,
// same wave-order sums and epilogues as gemm_os_body: the results are bit-identical.
template <int DT, int EPI, int XF, int MT, int NT, int KPW>
__device__ __forceinline__ void gemm_os_direct_body(const GemmP& a, int bx, int by, int bz, int gy, unsigned char* smem) {
  constexpr int NW = 8;
  constexpr int UNITS = (EPI == EPI_SILU_PAIR ? NT / 2 : NT) * MT;
  static_assert(UNITS <= NW, "one epilogue unit per wave");
  __shared__ float inv_s[32];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = bz * 16 * MT, mlast = a.M - 1;  // m-chunks of 16 MT rows
  const int t0 = bx * NT;
  const int kb = by * a.kps;  // first k step of the split
  const int kq = a.kps / NW, kr = a.kps % NW;
  const int ws = kq * w + min(w, kr), wn = kq + (w < kr ? 1 : 0);  // this wave's k steps [ws, ws + wn)

  // A wave may have at most 63 loads outstanding, and a load waits for every older one.  With the norm
  // transform the activation path (KPW x MT fragments, 12 sums-of-squares loads, one norm-weight chunk)
  // goes first, then the weights.  A wave's load instructions issue only as fast as its compute unit
  // takes data in, so a wave that requested gate_up's 36 weight blocks at once sat in that issue until
  // most of them had arrived (about 9 us, per-wave clock marks in a probe build) and only then reached
  // the transform, which ran after the stream instead of during it: a wide slice is requested in two
  // parts, the first W1 k steps (12 blocks) before the transform and the rest after it.  Without the
  // transform, a wide slice (down's 20 blocks) goes first and the fragments arrive while it streams.
  constexpr bool W_FIRST = XF != XF_RMS && NT * KPW > 16;
  constexpr int W1 = XF == XF_RMS && NT * KPW > 16 ? (12 + NT - 1) / NT : KPW;
  u32x4 A[KPW][NT];
  auto issue_w = [&](int s0, int s1) {
#pragma unroll
    for (int s = 0; s < KPW; ++s)
      if (s >= s0 && s < s1)
#pragma unroll
        for (int j = 0; j < NT; ++j)
          A[s][j] = FD_WLOAD(wblock(a.W, a.KS, t0 + j, kb + ws + min(s, max(wn, 1) - 1)));
  };
  if constexpr (W_FIRST) issue_w(0, KPW);
  // 1. the activation path: the wave's fragments, the rows' sums of squares (threads 0 .. 255: row
  //    tid / 8, tiles tid % 8 + 8q) and the split's norm weights (one 16-byte chunk per thread)
  u32x4 X[KPW][MT];
#pragma unroll
  for (int s = 0; s < KPW; ++s)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      // row-major: the row (clamped to the last; rows past it are never stored); fragment order: the
      // whole 1 KB block (m0 = 0)
      const int m = min(m0 + 16 * mt + lr, mlast), ks = kb + ws + min(s, max(wn, 1) - 1);
      const size_t off = a.xfrag ? (size_t)((2 * ks + (m0 >> 4) + mt) * 64 + lane) * 8 : (size_t)m * a.ldx + 32 * ks + 8 * lg;
      X[s][mt] = *reinterpret_cast<const u32x4*>(a.X + off);
    }
  constexpr int SQ = 12;  // unrolled sums-of-squares loads (96 tiles: hidden 1536); the rest in a loop
  __shared__ u32x4 nw_s[XF == XF_RMS ? 8 * KPW * 4 : 1];
  float ssv[SQ];
  u32x4 nwv = {0u, 0u, 0u, 0u};
  const bool nw_ld = XF == XF_RMS && (int)threadIdx.x < a.kps * 4;  // kps <= 8 KPW (the plan's bound)
  if constexpr (XF == XF_RMS) {
    if (threadIdx.x < 256) {
      const int m = m0 + (threadIdx.x >> 3), pp = threadIdx.x & 7;
#pragma unroll
      for (int q = 0; q < SQ; ++q) {
        const int t = pp + 8 * q;
        ssv[q] = (m < a.M && t < a.ssq_tiles) ? a.ssq[(size_t)t * a.ssq_ld + m] : 0.f;
      }
    }
    if (nw_ld) nwv = *reinterpret_cast<const u32x4*>(a.nw + 32 * kb + 8 * threadIdx.x);
  }
  // 2. the weight slice: KPW k steps x NT tiles per wave, all requested at once (with the transform, its
  //    first W1 steps)
  if constexpr (!W_FIRST) issue_w(0, W1);

  // 3. 1 / rms of the chunk's rows (gemm_os_body's order), then the transform in registers
  if constexpr (XF == XF_RMS) {
    if (nw_ld) nw_s[threadIdx.x] = nwv;
    if (threadIdx.x < 256) {
      float ss = 0.f;
#pragma unroll
      for (int q = 0; q < SQ; ++q) ss += ssv[q];
      const int m = m0 + (threadIdx.x >> 3), pp = threadIdx.x & 7;
      for (int q = SQ; pp + 8 * q < a.ssq_tiles; ++q) ss += (m < a.M) ? a.ssq[(size_t)(pp + 8 * q) * a.ssq_ld + m] : 0.f;
      ss += __shfl_xor(ss, 1, WAVE);
      ss += __shfl_xor(ss, 2, WAVE);
      ss += __shfl_xor(ss, 4, WAVE);
      if (pp == 0) inv_s[threadIdx.x >> 3] = 1.0f / sqrtf(ss / (float)a.H + a.eps);
    }
    __syncthreads();
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const float inv = inv_s[16 * mt + lr];
#pragma unroll
      for (int s = 0; s < KPW; ++s) X[s][mt] = xform<DT, XF>(X[s][mt], nw_s[(ws + min(s, max(wn, 1) - 1)) * 4 + lg], inv);
    }
  }
  if constexpr (!W_FIRST && W1 < KPW) {
    __builtin_amdgcn_sched_barrier(0);  // not hoisted above the transform
    issue_w(W1, KPW);
  }

  // 4. multiply
  f32x4 acc[NT][MT];
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[j][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < KPW; ++s) {
    if (s < wn) {
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[j][mt] = mfma16<DT>(A[s][j], X[s][mt], acc[j][mt]);
    }
  }

  // 5. the waves' partials, summed per unit in wave order
  f32x4* red = reinterpret_cast<f32x4*>(smem);  // [NW][NT][MT][64]
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[((w * NT + j) * MT + mt) * 64 + lane] = acc[j][mt];
  __syncthreads();
  constexpr int TPU = EPI == EPI_SILU_PAIR ? 2 : 1;  // tiles per unit
  f32x4 v[TPU] = {};
  const int u = w;
  const bool has_unit = u < UNITS;
  const int ut = (u / MT) * TPU, umt = u % MT;
  if (has_unit) {
#pragma unroll
    for (int q = 0; q < TPU; ++q) {
      f32x4 sum = red[((0 * NT + ut + q) * MT + umt) * 64 + lane];
      for (int ww = 1; ww < NW; ++ww) sum += red[((ww * NT + ut + q) * MT + umt) * 64 + lane];
      v[q] = sum;
    }
  }

  // 6. cross-workgroup k splits: the unit's partial, summed by the epilogue body (a separate launch), or,
  //    with a.gw, inside this launch: the tile group's splits meet at its counter and unit u of the group
  //    is summed by wave u / gy of split u % gy, in split order (gemm_os_epilogue_body's arithmetic)
  if (gy > 1) {
    const size_t grp = (size_t)bz * a.ngroups + bx;
    constexpr int per = NT * MT * 64;
    f32x4* part = reinterpret_cast<f32x4*>(a.part) + (grp * gy + by) * per;
    if (a.gw.cnt == nullptr) {
      if (has_unit) {
#pragma unroll
        for (int q = 0; q < TPU; ++q) part[((ut + q) * MT + umt) * 64 + lane] = v[q];
      }
      return;
    }
    if (has_unit) {
      const CohBuf pb = coh_buf(part, per * 16);
#pragma unroll
      for (int q = 0; q < TPU; ++q) coh_stf4(pb, (unsigned)(((ut + q) * MT + umt) * 64 + lane) * 16u, v[q]);
    }
    __shared__ int ok_s;
    if (threadIdx.x == 0) group_clear_other(a.gw, (int)((bz * gy + by) * a.ngroups + bx));
    if (!group_arrive_wait(a.gw, (int)grp, (unsigned)gy, &ok_s)) return;
    const CohBuf gb = coh_buf(reinterpret_cast<const f32x4*>(a.part) + grp * gy * per, (unsigned)(gy * per * 16));
    for (int u = w * gy + by; u < UNITS; u += NW * gy) {
      const int sut = (u / MT) * TPU, sumt = u % MT;
      f32x4 sv[TPU];
#pragma unroll
      for (int q = 0; q < TPU; ++q) {
        constexpr int SB = 16;
        const unsigned o = (unsigned)(((sut + q) * MT + sumt) * 64 + lane) * 16u;
        f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int y0 = 0; y0 < gy; y0 += SB) {
          f32x4 pv[SB];
#pragma unroll
          for (int y = 0; y < SB; ++y) pv[y] = coh_ldf4(gb, (unsigned)min(y0 + y, gy - 1) * (per * 16u) + o);
#pragma unroll
          for (int y = 0; y < SB; ++y)
            if (y0 + y < gy) sum = (y0 + y == 0) ? pv[y] : sum + pv[y];
        }
        sv[q] = sum;
      }
      os_epilogue<DT, EPI, TPU, false>(a, sv, m0 + 16 * sumt + lr, t0 + sut, lg);
    }
    return;
  }
  if (has_unit) os_epilogue<DT, EPI, TPU, false>(a, v, m0 + 16 * umt + lr, t0 + ut, lg);
}

template <int DT, int EPI, int XF, int MT, int NT, int KPW>
__global__ __launch_bounds__(512) void gemm_os_kernel(GemmP a) {
  extern __shared__ __align__(16) unsigned char smem[];
  if constexpr (NT <= 4) {
    gemm_os_direct_body<DT, EPI, XF, MT, NT, KPW>(a, blockIdx.x, blockIdx.y, blockIdx.z, gridDim.y, smem);
  } else if constexpr (EPI == EPI_SILU_PAIR) {
    // gate_up: every pair's MFMAs with the fragments in registers, then one pass of wave sums through LDS
    // and the pairs' SiLU * up by waves 0 .. NT / 2 x MT - 1 in parallel (no k split at the 1.5B shape);
    // a k split takes the LDS-staged body
    if (gridDim.y == 1)
      gemm_os_direct_body<DT, EPI, XF, MT, NT, KPW>(a, blockIdx.x, 0, blockIdx.z, 1, smem);
    else
      gemm_os_body<DT, EPI, XF, MT, NT, KPW, false>(a, blockIdx.x, blockIdx.y, blockIdx.z, gridDim.y, smem);
  } else {
    gemm_os_body<DT, EPI, XF, MT, NT, KPW, false>(a, blockIdx.x, blockIdx.y, blockIdx.z, gridDim.y, smem);
  }
}

// Sum of the k-split partials of one unit per wave, in split order, then the epilogue (workgroup =
// tile group bx of m-chunk bz; tid = threadIdx.x).
template <int DT, int EPI, int MT, int NT, bool COH>
__device__ __forceinline__ void gemm_os_epilogue_body(const GemmP& a, int splits, int bx, int bz, int tid) {
  constexpr int TPU = EPI == EPI_SILU_PAIR ? 2 : 1;
  constexpr int UNITS = NT / TPU * MT;
  const int lane = tid & 63, u = tid >> 6;
  if (u >= UNITS) return;
  const int lr = lane & 15, lg = lane >> 4;
  const int ut = (u / MT) * TPU, umt = u % MT;
  const size_t grp = (size_t)bz * a.ngroups + bx;
  constexpr int per = NT * MT * 64;
  const f32x4* part = reinterpret_cast<const f32x4*>(a.part) + grp * splits * per;
  f32x4 v[TPU];
#pragma unroll
  for (int q = 0; q < TPU; ++q) {
    const size_t o = ((ut + q) * MT + umt) * 64 + lane;
    constexpr int SB = 16;
    f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int y0 = 0; y0 < splits; y0 += SB) {
      f32x4 pv[SB];
#pragma unroll
      for (int y = 0; y < SB; ++y) pv[y] = ldf4<COH>(part + (size_t)min(y0 + y, splits - 1) * per + o);
#pragma unroll
      for (int y = 0; y < SB; ++y)
        if (y0 + y < splits) sum = (y0 + y == 0) ? pv[y] : sum + pv[y];
    }
    v[q] = sum;
  }
  os_epilogue<DT, EPI, TPU, COH>(a, v, bz * 16 * MT + 16 * umt + lr, bx * NT + ut, lg);
}

template <int DT, int EPI, int MT, int NT>
__global__ __launch_bounds__(512) void gemm_os_epilogue_kernel(GemmP a, int splits) {
  gemm_os_epilogue_body<DT, EPI, MT, NT, false>(a, splits, blockIdx.x, blockIdx.z, threadIdx.x);
}

}  // namespace fdllm
