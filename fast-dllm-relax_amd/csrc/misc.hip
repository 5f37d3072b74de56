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

// FastDLLMRMSNorm (cuda.py:269-275) from the producer's sums of squares: fp32 mean of squares,
// x * 1/sqrt(var + eps) cast to the model dtype, then the weight multiply in the model dtype.
template <int DT>
__global__ __launch_bounds__(256) void norm_rows_kernel(const u16* h, int hidden, const float* ssq, int ssq_ld,
                                                        const u16* w, float eps, u16* y, int hfrag, int yblk) {
  __shared__ float part_s[4];
  const int r = blockIdx.x;
  float ss = 0.f;
  for (int t = threadIdx.x; t < hidden / 16; t += 256) ss += ssq[(size_t)t * ssq_ld + r];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part_s[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float inv = 1.0f / sqrtf(((part_s[0] + part_s[1]) + (part_s[2] + part_s[3])) / (float)hidden + eps);
  for (int c = threadIdx.x; c < hidden; c += 256) {
    const u16 hv = h[hfrag ? frag_off(r, c) : (size_t)r * hidden + c];
    y[yblk ? frag_blk_off(r, c, hidden / 32) : (size_t)r * hidden + c] =
        from_f32<DT>(to_f32<DT>(w[c]) * rnd<DT>(to_f32<DT>(hv) * inv));
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
  if ((hfrag && rows > 32) || (yblk && hidden % 32)) return hipErrorInvalidValue;
  if (dt == DT_BF16)
    hipLaunchKernelGGL(norm_rows_kernel<DT_BF16>, dim3(rows), dim3(256), 0, st, h, hidden, ssq, ssq_ld, w, eps, y, hfrag,
                       yblk);
  else
    hipLaunchKernelGGL(norm_rows_kernel<DT_F16>, dim3(rows), dim3(256), 0, st, h, hidden, ssq, ssq_ld, w, eps, y, hfrag,
                       yblk);
  return hipGetLastError();
}

}  // namespace fdllm
