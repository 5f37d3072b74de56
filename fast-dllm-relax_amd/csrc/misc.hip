// Row kernels of the cached step: embedding gather, residual-stream load, final RMSNorm.
#include "common.hpp"
#include "kernels.hpp"

namespace fdllm {

// embed (fast_dllm_relax/model/cuda.py:698-699): out[r] = table[ids[r]]; ids outside the vocab are
// an error the host checks before the launch, so they are clamped here only to stay in bounds.
__global__ __launch_bounds__(256) void embed_kernel(const int32_t* ids, const u16* table, int vocab, int hidden,
                                                     u16* out) {
  const int r = blockIdx.x;
  int id = ids[r];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  const u32x4* src = reinterpret_cast<const u32x4*>(table + (size_t)id * hidden);
  u32x4* dst = reinterpret_cast<u32x4*>(out + (size_t)r * hidden);
  for (int c = threadIdx.x; c < hidden / 8; c += blockDim.x) dst[c] = src[c];
}

// The residual stream h starts as a copy of the input rows; each thread of the first H / 16 also
// leaves the sum of squares of one 16-column tile of its row for the first layer's RMSNorm (the
// layers' own residual epilogues leave the same statistics for the next norm).
template <int DT>
__global__ __launch_bounds__(256) void load_rows_kernel(const u16* x, int hidden, u16* h, float* ssq, int ssq_ld,
                                                        int hfrag) {
  const int r = blockIdx.x;
  const u32x4* src = reinterpret_cast<const u32x4*>(x + (size_t)r * hidden);
  for (int c = threadIdx.x; c < hidden / 8; c += blockDim.x)
    *reinterpret_cast<u32x4*>(h + (hfrag ? frag_off(r, 8 * c) : (size_t)r * hidden + 8 * c)) = src[c];
  for (int t = threadIdx.x; t < hidden / 16; t += blockDim.x) {
    const u32x4 a = src[2 * t], b = src[2 * t + 1];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float a0 = lo_f32<DT>(a[c]), a1 = hi_f32<DT>(a[c]);
      ss += a0 * a0;
      ss += a1 * a1;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float b0 = lo_f32<DT>(b[c]), b1 = hi_f32<DT>(b[c]);
      ss += b0 * b0;
      ss += b1 * b1;
    }
    ssq[(size_t)t * ssq_ld + r] = ss;
  }
}

// One normalised element, w * rnd(x * inv) rounded to the model dtype.  Each element is computed on its
// own (an empty asm on the result): for fp16 the compiler rounds x * inv either by an fp32 multiply and
// a conversion or by one mixed-precision fma (v_fma_mixlo_f16, a single rounding), and with eight
// elements in flight it mixed the two, which changed results against the one-element-per-thread form
// the rest of the build compiles to.
template <int DT>
__device__ __forceinline__ u16 norm_elem(float w, float x, float inv) {
  u16 r = from_f32<DT>(w * rnd<DT>(x * inv));
  asm volatile("" : "+v"(r));
  return r;
}

// FastDLLMRMSNorm (cuda.py:269-275) from the producer's sums of squares: fp32 mean of squares,
// x * 1/sqrt(var + eps) cast to the model dtype, then the weight multiply in the model dtype.
// A workgroup normalises 4 rows, one per wave.  A row's sum of squares is the sum of its per-16-column
// tile sums in a fixed order: four partial sums P_q (q = 0..3), P_q adding tiles 64 q + l + 256 j (j in
// order) in lane l and then a butterfly over the 64 lanes, and the total (P_0 + P_1) + (P_2 + P_3).  The
// rows then move in 16-byte units of 8 columns (consecutive threads take consecutive rows of one column
// group): read from h (row-major, or fragment order with hfrag), written row-major or, with yblk, in the
// large-M GEMMs' 1 KB fragment blocks.
template <int DT>
__global__ __launch_bounds__(256) void norm_rows_kernel(const u16* h, int rows, int hidden, const float* ssq,
                                                        int ssq_ld, const u16* w, float eps, u16* y, int hfrag,
                                                        int yblk) {
  constexpr int RPW = 4;  // rows per workgroup
  __shared__ float inv_s[RPW];
  const int r0 = blockIdx.x * RPW;
  const int ntiles = hidden / 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (r0 + wave < rows) {
    const int m = r0 + wave;
    float part[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float v = 0.f;
      for (int t = 64 * q + lane; t < ntiles; t += 256) v += ssq[(size_t)t * ssq_ld + m];
      part[q] = 64 * q < ntiles ? wave_sum(v) : 0.f;
    }
    if (lane == 0) inv_s[wave] = 1.0f / sqrtf(((part[0] + part[1]) + (part[2] + part[3])) / (float)hidden + eps);
  }
  __syncthreads();
  const int ks = hidden / 32;  // k steps (fragment blocks per 16-row block)
  for (int u = threadIdx.x; u < RPW * (hidden / 8); u += 256) {
    const int rl = u % RPW, c = 8 * (u / RPW);
    const int r = r0 + rl;
    if (r >= rows) continue;
    const float inv = inv_s[rl];
    const u32x4 hv = *reinterpret_cast<const u32x4*>(h + (hfrag ? frag_off(r, c) : (size_t)r * hidden + c));
    const u32x4 wv = *reinterpret_cast<const u32x4*>(w + c);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = pack2(norm_elem<DT>(lo_f32<DT>(wv[e]), lo_f32<DT>(hv[e]), inv),
                   norm_elem<DT>(hi_f32<DT>(wv[e]), hi_f32<DT>(hv[e]), inv));
    *reinterpret_cast<u32x4*>(y + (yblk ? frag_blk_off(r, c, ks) : (size_t)r * hidden + c)) = o;
  }
}

// The k-split sum + residual epilogue of an EPI_RESID projection (o_proj / down in a batched or
// prefill-sized call) fused with the next RMSNorm.  The split sums come row-major (part[split][rows][hidden],
// a part_rows GEMM launch).  A workgroup owns RPW rows.  Each 4-column unit adds its splits in split order
// (the requests of up to eight splits issued together), forms h = rnd(h + rnd(sum)) and the unit's sum of
// squares as the split-sum kernel's epilogue does; a 16-column tile's sum is (g0 + g1) + (g2 + g3) of its
// four units, again as there; h and the tile sums are written, and the rows are normalised exactly as
// norm_rows_kernel does, from the same sums (kept in LDS with the new rows), into y (row-major, or with
// yblk the large-M GEMMs' fragment blocks).
template <int DT>
__global__ __launch_bounds__(256) void resid_norm_kernel(const float* part, int splits, int rows, int hidden, u16* h,
                                                         float* ssq, int ssq_ld, const u16* w, float eps, u16* y,
                                                         int yblk) {
  constexpr int RPW = 2;                // rows per workgroup
  constexpr int MAXH = 2048;            // hidden sizes up to this (the launcher checks)
  constexpr int SB = 8;                 // split sums requested at once
  __shared__ float gss[RPW][MAXH / 4];
  __shared__ float tss[RPW][MAXH / 16];
  __shared__ __align__(16) u16 hl[RPW][MAXH];
  __shared__ float inv_s[RPW];
  const int r0 = blockIdx.x * RPW;
  const int nunits = hidden / 4, ntiles = hidden / 16;
  for (int u = threadIdx.x; u < RPW * nunits; u += 256) {
    const int rl = u / nunits, n = 4 * (u - rl * nunits), m = r0 + rl;
    if (m >= rows) continue;
    f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < splits; s0 += SB) {
      f32x4 v[SB];
#pragma unroll
      for (int q = 0; q < SB; ++q)
        v[q] = s0 + q < splits ? *reinterpret_cast<const f32x4*>(part + ((size_t)(s0 + q) * rows + m) * hidden + n)
                               : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < SB; ++q)
        if (s0 + q < splits) sum = s0 + q == 0 ? v[q] : sum + v[q];
    }
    u16* hp = h + (size_t)m * hidden + n;
    const u32x2 hv = *reinterpret_cast<const u32x2*>(hp);
    const float hf[4] = {lo_f32<DT>(hv[0]), hi_f32<DT>(hv[0]), lo_f32<DT>(hv[1]), hi_f32<DT>(hv[1])};
    u16 out[4];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[i] = from_f32<DT>(hf[i] + rnd<DT>(sum[i]));
      const float yv = to_f32<DT>(out[i]);
      ss += yv * yv;
    }
    const u32x2 o = u32x2{pack2(out[0], out[1]), pack2(out[2], out[3])};
    *reinterpret_cast<u32x2*>(hp) = o;
    *reinterpret_cast<u32x2*>(&hl[rl][n]) = o;
    gss[rl][n / 4] = ss;
  }
  __syncthreads();
  for (int u = threadIdx.x; u < RPW * ntiles; u += 256) {
    const int rl = u / ntiles, t = u - rl * ntiles, m = r0 + rl;
    if (m >= rows) continue;
    const float ts = (gss[rl][4 * t] + gss[rl][4 * t + 1]) + (gss[rl][4 * t + 2] + gss[rl][4 * t + 3]);
    ssq[(size_t)t * ssq_ld + m] = ts;
    tss[rl][t] = ts;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (wave < RPW && r0 + wave < rows) {
    float pq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float v = 0.f;
      for (int t = 64 * q + lane; t < ntiles; t += 256) v += tss[wave][t];
      pq[q] = 64 * q < ntiles ? wave_sum(v) : 0.f;
    }
    if (lane == 0) inv_s[wave] = 1.0f / sqrtf(((pq[0] + pq[1]) + (pq[2] + pq[3])) / (float)hidden + eps);
  }
  __syncthreads();
  const int ks = hidden / 32;
  for (int u = threadIdx.x; u < RPW * (hidden / 8); u += 256) {
    const int rl = u % RPW, c = 8 * (u / RPW);
    const int r = r0 + rl;
    if (r >= rows) continue;
    const float inv = inv_s[rl];
    const u32x4 hv = *reinterpret_cast<const u32x4*>(&hl[rl][c]);
    const u32x4 wv = *reinterpret_cast<const u32x4*>(w + c);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = pack2(norm_elem<DT>(lo_f32<DT>(wv[e]), lo_f32<DT>(hv[e]), inv),
                   norm_elem<DT>(hi_f32<DT>(wv[e]), hi_f32<DT>(hv[e]), inv));
    *reinterpret_cast<u32x4*>(y + (yblk ? frag_blk_off(r, c, ks) : (size_t)r * hidden + c)) = o;
  }
}

// RoPE tables of one call (cuda.py:288-299): position pos_offset + r, inv_freq = exp(-ln(theta) * i / 64),
// angle = pos * inv_freq in fp32, cos / sin in fp32 rounded to the model dtype (emb = [f, f], so one
// entry serves dims i and i + 64).  Shared by every layer's attention.
template <int DT>
__global__ __launch_bounds__(64) void rope_table_kernel(const int32_t* pos_offset, int rows_per_seq, float nlt,
                                                        float* tab) {
  const int r = blockIdx.x, i = threadIdx.x;
  const int b = r / rows_per_seq;
  const float pos = (float)(pos_offset[b] + (r - b * rows_per_seq));
  const float fr = pos * expf((nlt * (float)i) / 64.0f);
  tab[((size_t)r * 64 + i) * 2] = rnd<DT>(cosf(fr));
  tab[((size_t)r * 64 + i) * 2 + 1] = rnd<DT>(sinf(fr));
}

// The cache write of fast_dllm.kv_write / attn_inplace (_write_rows, fast_dllm_relax/runtime.py:51-60):
// the k and v rows into their cache windows in one launch, 16 bytes per thread and tensor (a copy: the
// bytes are the caller's).  The host takes this path when every pointer and the size are 16-byte
// multiples.
__global__ __launch_bounds__(256) void kv_copy_kernel(const u32x4* k, const u32x4* v, u32x4* kd, u32x4* vd, int n16) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n16) {
    kd[i] = k[i];
    vd[i] = v[i];
  }
}

hipError_t launch_kv_copy(const void* k, const void* v, void* kd, void* vd, size_t bytes, hipStream_t st) {
  const int n16 = (int)(bytes / 16);
  hipLaunchKernelGGL(kv_copy_kernel, dim3((n16 + 255) / 256), dim3(256), 0, st, (const u32x4*)k, (const u32x4*)v,
                     (u32x4*)kd, (u32x4*)vd, n16);
  return hipGetLastError();
}

hipError_t launch_embed(const int32_t* ids, int n, const uint16_t* table, int vocab, int hidden, uint16_t* out,
                        hipStream_t st) {
  hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(256), 0, st, ids, table, vocab, hidden, out);
  return hipGetLastError();
}

hipError_t launch_load_rows(int dt, const uint16_t* x, int rows, int hidden, uint16_t* h, float* ssq, int ssq_ld,
                            hipStream_t st, int hfrag) {
  if (hfrag && rows > 32) return hipErrorInvalidValue;
  if (dt == DT_BF16)
    hipLaunchKernelGGL(load_rows_kernel<DT_BF16>, dim3(rows), dim3(256), 0, st, x, hidden, h, ssq, ssq_ld, hfrag);
  else
    hipLaunchKernelGGL(load_rows_kernel<DT_F16>, dim3(rows), dim3(256), 0, st, x, hidden, h, ssq, ssq_ld, hfrag);
  return hipGetLastError();
}

hipError_t launch_rope_table(int dt, const int32_t* pos_offset, int rows, int rows_per_seq, float neg_log_theta, float* tab,
                             hipStream_t st) {
  if (dt == DT_BF16)
    hipLaunchKernelGGL(rope_table_kernel<DT_BF16>, dim3(rows), dim3(64), 0, st, pos_offset, rows_per_seq, neg_log_theta,
                       tab);
  else
    hipLaunchKernelGGL(rope_table_kernel<DT_F16>, dim3(rows), dim3(64), 0, st, pos_offset, rows_per_seq, neg_log_theta,
                       tab);
  return hipGetLastError();
}

hipError_t launch_norm_rows(int dt, const uint16_t* h, int rows, int hidden, const float* ssq, int ssq_ld,
                            const uint16_t* w, float eps, uint16_t* y, hipStream_t st, int hfrag, int yblk) {
  if ((hfrag && rows > 32) || hidden % 32) return hipErrorInvalidValue;
  const int wgs = (rows + 3) / 4;
  if (dt == DT_BF16)
    hipLaunchKernelGGL(norm_rows_kernel<DT_BF16>, dim3(wgs), dim3(256), 0, st, h, rows, hidden, ssq, ssq_ld, w, eps, y,
                       hfrag, yblk);
  else
    hipLaunchKernelGGL(norm_rows_kernel<DT_F16>, dim3(wgs), dim3(256), 0, st, h, rows, hidden, ssq, ssq_ld, w, eps, y,
                       hfrag, yblk);
  return hipGetLastError();
}

hipError_t launch_resid_norm(int dt, const float* part, int splits, int rows, int hidden, uint16_t* h, float* ssq,
                             int ssq_ld, const uint16_t* w, float eps, uint16_t* y, int yblk, hipStream_t st) {
  if (hidden % 32 || hidden > 2048 || splits < 1) return hipErrorInvalidValue;
  const int wgs = (rows + 1) / 2;
  if (dt == DT_BF16)
    hipLaunchKernelGGL(resid_norm_kernel<DT_BF16>, dim3(wgs), dim3(256), 0, st, part, splits, rows, hidden, h, ssq, ssq_ld,
                       w, eps, y, yblk);
  else
    hipLaunchKernelGGL(resid_norm_kernel<DT_F16>, dim3(wgs), dim3(256), 0, st, part, splits, rows, hidden, h, ssq, ssq_ld,
                       w, eps, y, yblk);
  return hipGetLastError();
}

}  // namespace fdllm
