// Large-M GEMM over packed weights (prefill, stateless forward, batched steps): Y[M, N] = X[M, K] . W[N, K]^T
// on MFMA 16x16x32 with fp32 accumulation, same epilogues and rounding points as the skinny kernels.
//
// A workgroup computes a block of BM = 16 MF NWM rows by BN = 16 TPW NWN columns with NWM x NWN waves:
// wave (wm, wn) owns TPW consecutive 16-row weight tiles and MF row blocks.  Weight blocks go straight
// from global memory into registers (they are already in operand order); with NWM = 2 two waves load
// each (the second mostly from L1), in exchange for each wave reading only its own MF activation
// fragments from LDS instead of all of them.
//
// The k loop runs in stages of KSS k steps.  Activations pass through two LDS buffers in MFMA fragment
// order: while stage s is multiplied out of one buffer, stage s + 1 is loaded into registers and then
// normalised (XF_RMS) and stored into the other.  The weight blocks go to WD + 1 register buffers:
// those of stage s + WD are requested at the start of stage s.  Every load is unconditional (stages past
// the last one re-read the last), so the compiler's wait counts stay exact.
//
// K splits (gridDim.y > 1, for launches with too few blocks to fill the chip): split y runs its own
// range of stages and stores its fp32 sums per (tile, 16-row block) unit; gemm_mm_split_epilogue_kernel
// adds them in split order and applies the epilogue, so results stay deterministic.
//
// Workgroup order: the launch has 8 x per workgroups; workgroup b runs block (b % 8) * per + b / 8 in a
// column-major block order, so consecutive blocks of one weight column block land on the same XCD (the
// hardware deals workgroups to the 8 XCDs round-robin) and share that XCD's L2.
#pragma once
#include "gemm_body.hpp"

namespace fdllm {

template <int DT, int EPI, int XF, int MF, int TPW, int NWM, int NWN, int KSS, int WD>
__global__ __launch_bounds__(64 * NWM * NWN) void gemm_mm_kernel(GemmP a, int nbm, int nbn) {
  constexpr int NW = NWM * NWN;
  constexpr int MFT = MF * NWM;                // row blocks of the workgroup
  constexpr int BM = 16 * MFT;
  constexpr int NT = 64 * NW;                  // threads
  constexpr int XCH = KSS * MFT * 64 / NT;     // activation chunks (16 bytes) per thread per stage
  static_assert(KSS * MFT % NW == 0, "whole fragment blocks per wave");
  static_assert(NT % BM == 0 && BM <= NT, "threads per row for the norm prologue");
  static_assert(EPI != EPI_SILU_PAIR || TPW % 2 == 0, "gate/up pairs stay within a wave");
  static_assert(EPI != EPI_LOGITS || TPW * NWN == 16, "one 256-column confidence tile per block column");
  extern __shared__ __align__(16) unsigned char smem[];
  u32x4* xl = reinterpret_cast<u32x4*>(smem);  // [2][KSS][MFT][64]
  __shared__ float inv_s[BM];

  const int total = nbm * nbn;
  const int per = (total + 7) / 8;
  const int logical = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (logical >= total) return;
  const int nb = logical / nbm, mb = logical - nb * nbm;

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w / NWN, wn = w - wm * NWN;
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = mb * BM, mlast = a.M - 1;
  const int f0 = wm * MF;                      // this wave's first row block
  const int t0 = (nb * NWN + wn) * TPW;
  const int nst = a.KS / KSS / (int)gridDim.y;  // stages of this k split
  const int kb = (int)blockIdx.y * nst * KSS;   // its first k step

  // 1 / rms of the block's rows from the producer's per-16-column sums of squares
  if constexpr (XF == XF_RMS) {
    constexpr int TPR = NT / BM;
    const int r = threadIdx.x / TPR, pp = threadIdx.x % TPR;
    const int m = m0 + r;
    float ss = 0.f;
    if (m < a.M)
      for (int t = pp; t < a.ssq_tiles; t += TPR) ss += a.ssq[(size_t)t * a.ssq_ld + m];
#pragma unroll
    for (int o = 1; o < TPR; o <<= 1) ss += __shfl_xor(ss, o, WAVE);
    if (pp == 0) inv_s[r] = 1.0f / sqrtf(ss / (float)a.H + a.eps);
    __syncthreads();
  }

  // chunk i of this thread: fragment block (ks, f) = w + NW i, lane = this lane
  u32x4 xr[XCH];
  auto xload = [&](int st) {
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int blk = w + NW * i, ks = blk / MFT, f = blk - ks * MFT;
      const int m = min(m0 + 16 * f + lr, mlast);
      const int k = 32 * (kb + st * KSS + ks) + 8 * lg;
      xr[i] = *reinterpret_cast<const u32x4*>(a.X + (size_t)m * a.ldx + k);
    }
  };
  auto xstore = [&](int buf, int st) {
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int blk = w + NW * i, ks = blk / MFT, f = blk - ks * MFT;
      u32x4 v = xr[i];
      if constexpr (XF == XF_RMS) {
        const int k = 32 * (kb + st * KSS + ks) + 8 * lg;
        v = xform<DT, XF>(v, *reinterpret_cast<const u32x4*>(a.nw + k), inv_s[16 * f + lr]);
      }
      xl[((buf * KSS + ks) * MFT + f) * 64 + lane] = v;
    }
  };
  // weight blocks: WD + 1 register buffers, stage s + WD requested while stage s is multiplied
  constexpr int NB = WD + 1;
  u32x4 wv[NB][KSS][TPW];
  const int tlast = a.ntiles - 1;
  auto wload = [&](int st, u32x4(&dst)[KSS][TPW]) {
#pragma unroll
    for (int ks = 0; ks < KSS; ++ks)
#pragma unroll
      for (int j = 0; j < TPW; ++j)
        dst[ks][j] = *wblock(a.W, a.KS, min(t0 + j, tlast), kb + st * KSS + ks);
  };
  f32x4 acc[TPW][MF];
#pragma unroll
  for (int j = 0; j < TPW; ++j)
#pragma unroll
    for (int f = 0; f < MF; ++f) acc[j][f] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int buf, const u32x4(&src)[KSS][TPW]) {
#pragma unroll
    for (int ks = 0; ks < KSS; ++ks) {
      u32x4 b[MF];
#pragma unroll
      for (int f = 0; f < MF; ++f) b[f] = xl[((buf * KSS + ks) * MFT + f0 + f) * 64 + lane];
#pragma unroll
      for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int f = 0; f < MF; ++f) acc[j][f] = mfma16<DT>(src[ks][j], b[f], acc[j][f]);
    }
  };

  xload(0);
#pragma unroll
  for (int d = 0; d < WD; ++d) wload(min(d, nst - 1), wv[d]);
  xstore(0, 0);
  __syncthreads();
  // stages run in rounds of NB so that buffer indices are compile-time; past the last stage the loads
  // repeat the last stage and nothing is multiplied
  for (int st0 = 0; st0 < nst; st0 += NB) {
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int st = st0 + q;
      const int sx = min(st + 1, nst - 1);
      xload(sx);
      wload(min(st + WD, nst - 1), wv[(q + WD) % NB]);
      if (st < nst) compute(st & 1, wv[q]);
      xstore((st + 1) & 1, sx);
      __syncthreads();
    }
  }

  if (gridDim.y > 1) {
    // this split's sums, unit by unit
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int f = 0; f < MF; ++f) store_split_unit(a, blockIdx.y, t0 + j, mb * MFT + f0 + f, lane, acc[j][f]);
    return;
  }

  // epilogue: one (tile or gate/up pair, 16-row block) unit at a time
  if constexpr (EPI == EPI_LOGITS) {
    // the block's logits, rounded to the model dtype as get_logits does (cuda.py:708-711), go to LDS
    // ([BM][256] model-dtype values; exact) and to the optional fp32 output; then one wave per row
    // reduces the row's 256 columns to the confidence statistics with the same lane order and
    // butterflies as the streaming kernel, so both give identical bits
    u16* tile = reinterpret_cast<u16*>(smem);
    const int n0 = nb * 256;
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int f = 0; f < MF; ++f) {
        const int ml = 16 * (f0 + f) + lr, nl = 16 * (wn * TPW + j) + 4 * lg, n = n0 + nl, m = m0 + ml;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = rnd<DT>(acc[j][f][i]);
        *reinterpret_cast<u32x2*>(tile + ml * 256 + nl) =
            u32x2{pack2(from_f32<DT>(v[0]), from_f32<DT>(v[1])), pack2(from_f32<DT>(v[2]), from_f32<DT>(v[3]))};
        if (a.logits != nullptr && m < a.M) {
          float* dst = a.logits + (size_t)m * a.ldl + n;
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
    logits_tile_stats<DT, BM, NW>(a, tile, m0, nb, w, lane);
  } else if constexpr (EPI == EPI_SILU_PAIR) {
#pragma unroll
    for (int p = 0; p < TPW / 2; ++p)
#pragma unroll
      for (int f = 0; f < MF; ++f) {
        const f32x4 v[2] = {acc[2 * p][f], acc[2 * p + 1][f]};
        os_epilogue<DT, EPI, 2, false>(a, v, m0 + 16 * (f0 + f) + lr, t0 + 2 * p, lg);
      }
  } else {
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int f = 0; f < MF; ++f) {
        const f32x4 v[1] = {acc[j][f]};
        os_epilogue<DT, EPI, 1, false>(a, v, m0 + 16 * (f0 + f) + lr, t0 + j, lg);
      }
  }
}

// Sum of the k-split partials of one unit per wave, in split order, then the epilogue: workgroup
// (unit x, 4 row blocks y); a unit is tile x, or gate/up pair x (tiles 2x, 2x + 1).
template <int DT, int EPI>
__global__ __launch_bounds__(256) void gemm_mm_split_epilogue_kernel(GemmP a, int splits) {
  constexpr int TPU = EPI == EPI_SILU_PAIR ? 2 : 1;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int nblk = (a.M + 15) / 16;
  const int b = (int)blockIdx.y * 4 + w;
  if (b >= nblk) return;
  const int t = (int)blockIdx.x * TPU;
  const f32x4* part = reinterpret_cast<const f32x4*>(a.part);
  f32x4 v[TPU];
#pragma unroll
  for (int q = 0; q < TPU; ++q) {
    f32x4 sum = part[((size_t)(t + q) * nblk + b) * 64 + lane];
    for (int y = 1; y < splits; ++y) sum += part[(((size_t)y * a.ntiles + t + q) * nblk + b) * 64 + lane];
    v[q] = sum;
  }
  os_epilogue<DT, EPI, TPU, false>(a, v, 16 * b + lr, t, lg);
}

template <int MF, int TPW, int NWM, int NWN, int KSS, int WD>
struct MmCfg {
  static constexpr int mf = MF, tpw = TPW, nwm = NWM, nwn = NWN, nw = NWM * NWN, kss = KSS, wd = WD;
  static constexpr int bm = 16 * MF * NWM, bn_tiles = TPW * NWN;
  static constexpr size_t lds = 2ull * KSS * MF * NWM * 64 * 16;
  static constexpr size_t lds_logits = (size_t)16 * MF * NWM * 256 * 2;  // EPI_LOGITS tile [BM][256] u16
};

}  // namespace fdllm
