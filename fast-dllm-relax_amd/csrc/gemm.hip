// Skinny projection GEMMs of the cached step: Y[M, N] = X[M, K] . W[N, K]^T, M <= 32 per m-chunk.
//
// The weights stream from HBM once; the activations of one k-slice sit in LDS.  Each wave owns TPW
// tiles of 16 weight rows and all m-chunk rows; per 32-wide k step a lane loads 16 contiguous bytes of
// one weight row (A operand) and 16 bytes of one activation row from LDS (B operand), so the MFMA
// produces C^T[n, m] and each lane ends with 4 consecutive output columns of one row.
// Split-K over gridDim.y: partials go to a workspace and the last workgroup of a column block to
// arrive sums them in split order (deterministic) and runs the epilogue.
//
// Epilogues follow the reference's rounding points (fast_dllm_relax/model/cuda.py):
//   EPI_STORE   y = rnd(acc)                                  o_proj alone, down alone
//   EPI_BIAS    y = rnd(acc + b[n])                           qkv_proj + bias (cuda.py:389-399)
//   EPI_RESID   y = rnd(r + rnd(acc))                         o_proj / down_proj + residual (cuda.py:577-578)
//   EPI_SILU    y = rnd(rnd(silu(rnd(g))) * rnd(u))           gate_up + _silu_fp32 * up (cuda.py:319-348)
//   EPI_LOGITS  logits fp32 = rnd(acc), plus per-256-column confidence tile statistics (cuda.py:704-711)
#include "common.hpp"
#include "kernels.hpp"

namespace fdllm {

template <int DT, int EPI, int TPW, int MT>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(GemmArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  u16* xs = reinterpret_cast<u16*>(smem_raw);
  __shared__ int last_flag;

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int kc = a.kc;
  const int k0 = blockIdx.y * kc;
  const int m0 = blockIdx.z * 16 * MT;
  const int xld = kc + 8;

  // stage the activation k-slice: rows m0 .. m0 + 16 MT (zero past M)
  {
    const int per_row = kc / 8;
    for (int idx = threadIdx.x; idx < 16 * MT * per_row; idx += 256) {
      int m = idx / per_row, c = idx - m * per_row;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (m0 + m < a.M) v = *reinterpret_cast<const u32x4*>(a.X + (size_t)(m0 + m) * a.ldx + k0 + c * 8);
      *reinterpret_cast<u32x4*>(xs + m * xld + c * 8) = v;
    }
  }

  const int row_base = blockIdx.x * a.wg_rows + w * 16;
  const u16* wp[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    int r = row_base + j * a.tile_stride + lr;
    r = r < a.N ? r : a.N - 1;
    wp[j] = a.W + (size_t)r * a.K + k0 + lg * 8;
  }
  __syncthreads();

  f32x4 acc[TPW][MT];
#pragma unroll
  for (int j = 0; j < TPW; ++j)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[j][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  constexpr int U = 4;  // k steps per group
  const int ng = kc / (32 * U);
  u32x4 A0[U][TPW], A1[U][TPW];
  auto load = [&](int g, u32x4(&dst)[U][TPW]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < TPW; ++j)
        dst[u][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wp[j] + (g * U + u) * 32));
  };
  auto comp = [&](int g, u32x4(&src)[U][TPW]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      u32x4 b[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        b[mt] = *reinterpret_cast<const u32x4*>(xs + (16 * mt + lr) * xld + (g * U + u) * 32 + lg * 8);
#pragma unroll
      for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[j][mt] = mfma16<DT>(src[u][j], b[mt], acc[j][mt]);
    }
  };
  load(0, A0);
  int g = 0;
  for (; g + 1 < ng; g += 2) {
    load(g + 1, A1);
    comp(g, A0);
    if (g + 2 < ng) load(g + 2, A0);
    comp(g + 1, A1);
  }
  if (g < ng) comp(g, A0);

  // ---- split-K fix-up ----
  if (gridDim.y > 1) {
    const size_t per_wg = (size_t)4 * TPW * MT * 64;  // f32x4 per workgroup
    const size_t grp = (size_t)blockIdx.z * gridDim.x + blockIdx.x;
    f32x4* part = reinterpret_cast<f32x4*>(a.partial) + (grp * gridDim.y) * per_wg;
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        part[blockIdx.y * per_wg + ((w * TPW + j) * MT + mt) * 64 + lane] = acc[j][mt];
    if (!arrive_last(a.counters + grp, gridDim.y, &last_flag)) return;
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        f32x4 s = part[((w * TPW + j) * MT + mt) * 64 + lane];
        for (int y = 1; y < (int)gridDim.y; ++y) s += part[y * per_wg + ((w * TPW + j) * MT + mt) * 64 + lane];
        acc[j][mt] = s;
      }
  }

  // ---- epilogues ----
  if constexpr (EPI == EPI_SILU) {
    // tile 0 = gate rows n, tile 1 = up rows n + tile_stride
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      int m = m0 + 16 * mt + lr;
      int n = row_base + 4 * lg;
      if (m >= a.M || n >= a.tile_stride) continue;
      u16 out[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float gt = rnd<DT>(acc[0][mt][i]);
        float up = rnd<DT>(acc[1][mt][i]);
        float s = rnd<DT>(gt * (1.0f / (1.0f + expf(-gt))));
        out[i] = from_f32<DT>(s * up);
      }
      u32x2 pk = {(uint32_t)out[0] | ((uint32_t)out[1] << 16), (uint32_t)out[2] | ((uint32_t)out[3] << 16)};
      *reinterpret_cast<u32x2*>(a.Y + (size_t)m * a.ldy + n) = pk;
    }
  } else if constexpr (EPI == EPI_LOGITS) {
    // logits (optional) and 256-column confidence tile statistics; one workgroup = one tile
    float* tile = reinterpret_cast<float*>(smem_raw);  // [16 MT][256], reuses the activation slice
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        int m = 16 * mt + lr;
        int nl = w * 16 + j * a.tile_stride + 4 * lg;  // column inside the 256-wide tile
        int n = blockIdx.x * a.wg_rows + nl;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = rnd<DT>(acc[j][mt][i]);
        *reinterpret_cast<f32x4*>(tile + m * 256 + nl) = f32x4{v[0], v[1], v[2], v[3]};
        if (a.logits != nullptr && m0 + m < a.M) {
          float* dst = a.logits + (size_t)(m0 + m) * a.ldl + n;
          if (n + 3 < a.N) {
            *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
          } else {
            for (int i = 0; i < 4; ++i)
              if (n + i < a.N) dst[i] = v[i];
          }
        }
      }
    if (a.stat_m == nullptr) return;
    __syncthreads();
    const int n0 = blockIdx.x * 256;
    const int tiles = a.stat_tiles;
    for (int m = w; m < 16 * MT; m += 4) {
      if (m0 + m >= a.M) break;
      const float* row = tile + m * 256;
      float vmax = -INFINITY;
      int amax = 0x7fffffff;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int c = lane + 64 * i;
        if (n0 + c < a.N) {
          float x = row[c];
          if (x > vmax) { vmax = x; amax = n0 + c; }
        }
      }
      for (int k = 32; k >= 1; k >>= 1) {
        float ov = __shfl_xor(vmax, k, WAVE);
        int oa = __shfl_xor(amax, k, WAVE);
        if (ov > vmax || (ov == vmax && oa < amax)) { vmax = ov; amax = oa; }
      }
      float s;
      {
#pragma clang fp contract(off)
        s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          int c = lane + 64 * i;
          if (n0 + c < a.N) s = s + fd_exp_neg(row[c] - vmax);
        }
        for (int k = 32; k >= 1; k >>= 1) s = s + __shfl_xor(s, k, WAVE);
      }
      if (lane == 0) {
        size_t o = (size_t)(m0 + m) * tiles + blockIdx.x;
        a.stat_m[o] = vmax;
        a.stat_a[o] = amax;
        a.stat_s[o] = s;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        int m = m0 + 16 * mt + lr;
        int n = row_base + j * a.tile_stride + 4 * lg;
        if (m >= a.M || n >= a.N) continue;
        u16 out[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = acc[j][mt][i];
          if constexpr (EPI == EPI_BIAS) {
            v = rnd<DT>(v + to_f32<DT>(a.bias[n + i]));
          } else if constexpr (EPI == EPI_RESID) {
            v = to_f32<DT>(a.resid[(size_t)m * a.ldr + n + i]) + rnd<DT>(v);
          }
          out[i] = from_f32<DT>(v);
        }
        u32x2 pk = {(uint32_t)out[0] | ((uint32_t)out[1] << 16), (uint32_t)out[2] | ((uint32_t)out[3] << 16)};
        *reinterpret_cast<u32x2*>(a.Y + (size_t)m * a.ldy + n) = pk;
      }
  }
}

// One wave per row: combine the tile statistics into (argmax, maxp) in the fixed lane order.
__global__ __launch_bounds__(64) void confidence_combine_kernel(const float* stat_m, const int32_t* stat_a,
                                                                const float* stat_s, int tiles, int rows,
                                                                int32_t* ids, float* maxp) {
#pragma clang fp contract(off)
  const int r = blockIdx.x, lane = threadIdx.x;
  if (r >= rows) return;
  const float* m = stat_m + (size_t)r * tiles;
  const int32_t* am = stat_a + (size_t)r * tiles;
  const float* s = stat_s + (size_t)r * tiles;
  float vmax = -INFINITY;
  int amax = 0x7fffffff;
  for (int t = lane; t < tiles; t += 64) {
    float x = m[t];
    if (x > vmax) { vmax = x; amax = am[t]; }
  }
  for (int k = 32; k >= 1; k >>= 1) {
    float ov = __shfl_xor(vmax, k, WAVE);
    int oa = __shfl_xor(amax, k, WAVE);
    if (ov > vmax || (ov == vmax && oa < amax)) { vmax = ov; amax = oa; }
  }
  float acc = 0.0f;
  for (int t = lane; t < tiles; t += 64) {
    float wgt = s[t] * fd_exp_neg(m[t] - vmax);
    acc = acc + wgt;
  }
  for (int k = 32; k >= 1; k >>= 1) acc = acc + __shfl_xor(acc, k, WAVE);
  if (lane == 0) {
    ids[r] = amax;
    maxp[r] = 1.0f / acc;
  }
}

// Tile statistics straight from an fp32 logits matrix [rows, ld] (confidence of given logits).
__global__ __launch_bounds__(64) void confidence_tiles_kernel(const float* logits, int ld, int vocab, int tiles,
                                                              float* stat_m, int32_t* stat_a, float* stat_s) {
#pragma clang fp contract(off)
  const int t = blockIdx.x, r = blockIdx.y, lane = threadIdx.x;
  const float* row = logits + (size_t)r * ld;
  const int n0 = t * 256;
  float vmax = -INFINITY;
  int amax = 0x7fffffff;
  for (int i = 0; i < 4; ++i) {
    int c = n0 + lane + 64 * i;
    if (c < vocab) {
      float x = row[c];
      if (x > vmax) { vmax = x; amax = c; }
    }
  }
  for (int k = 32; k >= 1; k >>= 1) {
    float ov = __shfl_xor(vmax, k, WAVE);
    int oa = __shfl_xor(amax, k, WAVE);
    if (ov > vmax || (ov == vmax && oa < amax)) { vmax = ov; amax = oa; }
  }
  float s = 0.0f;
  for (int i = 0; i < 4; ++i) {
    int c = n0 + lane + 64 * i;
    if (c < vocab) s = s + fd_exp_neg(row[c] - vmax);
  }
  for (int k = 32; k >= 1; k >>= 1) s = s + __shfl_xor(s, k, WAVE);
  if (lane == 0) {
    size_t o = (size_t)r * tiles + t;
    stat_m[o] = vmax;
    stat_a[o] = amax;
    stat_s[o] = s;
  }
}

// ---- launchers ---------------------------------------------------------------------------------
template <int DT, int EPI, int TPW, int MT>
static hipError_t launch_one(const GemmArgs& a, int nblocks, int ksplit, int mchunks, hipStream_t st) {
  size_t lds = (size_t)16 * MT * (a.kc + 8) * 2;
  if (EPI == EPI_LOGITS && lds < (size_t)16 * MT * 256 * 4) lds = (size_t)16 * MT * 256 * 4;
  auto kern = gemm_skinny_kernel<DT, EPI, TPW, MT>;
  static size_t attr_lds = 64 * 1024;  // the launch limit without the attribute
  if (lds > attr_lds) {
    // a runtime that needs no attribute for LDS up to the device limit may reject it: clear that
    // error and let the launch itself report whether the size fits
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      (void)hipGetLastError();
    attr_lds = lds;
  }
  hipLaunchKernelGGL(kern, dim3(nblocks, ksplit, mchunks), dim3(256), lds, st, a);
  return hipGetLastError();
}

template <int DT>
static hipError_t gemm_dispatch(int epi, int tpw, int mt, const GemmArgs& a, int nblocks, int ksplit, int mchunks,
                                hipStream_t st) {
#define FD_CASE(E, T, M_) \
  if (epi == E && tpw == T && mt == M_) return launch_one<DT, E, T, M_>(a, nblocks, ksplit, mchunks, st);
  FD_CASE(EPI_STORE, 2, 1) FD_CASE(EPI_STORE, 2, 2)
  FD_CASE(EPI_BIAS, 2, 1) FD_CASE(EPI_BIAS, 2, 2)
  FD_CASE(EPI_RESID, 2, 1) FD_CASE(EPI_RESID, 2, 2)
  FD_CASE(EPI_SILU, 2, 1) FD_CASE(EPI_SILU, 2, 2)
  FD_CASE(EPI_LOGITS, 4, 1) FD_CASE(EPI_LOGITS, 4, 2)
#undef FD_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_gemm(int dt, int epi, int tpw, int mt, const GemmArgs& a, int nblocks, int ksplit, int mchunks,
                       hipStream_t st) {
  if (dt == DT_BF16) return gemm_dispatch<DT_BF16>(epi, tpw, mt, a, nblocks, ksplit, mchunks, st);
  return gemm_dispatch<DT_F16>(epi, tpw, mt, a, nblocks, ksplit, mchunks, st);
}

hipError_t launch_confidence_combine(const float* sm, const int32_t* sa, const float* ss, int tiles, int rows,
                                     int32_t* ids, float* maxp, hipStream_t st) {
  hipLaunchKernelGGL(confidence_combine_kernel, dim3(rows), dim3(64), 0, st, sm, sa, ss, tiles, rows, ids, maxp);
  return hipGetLastError();
}

hipError_t launch_confidence_tiles(const float* logits, int ld, int vocab, int rows, float* sm, int32_t* sa,
                                   float* ss, hipStream_t st) {
  int tiles = (vocab + 255) / 256;
  hipLaunchKernelGGL(confidence_tiles_kernel, dim3(tiles, rows), dim3(64), 0, st, logits, ld, vocab, tiles, sm, sa, ss);
  return hipGetLastError();
}

}  // namespace fdllm
