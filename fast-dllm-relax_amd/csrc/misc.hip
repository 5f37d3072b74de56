// Row kernels of the cached step: embedding gather, RMSNorm, RoPE + KV-cache append.
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

// FastDLLMRMSNorm (cuda.py:269-275): fp32 mean of squares, x * 1/sqrt(var + eps) cast to the model
// dtype, then the weight multiply in the model dtype.
template <int DT>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const u16* x, int ldx, int hidden, const u16* w, float eps,
                                                      u16* y, int ldy) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const u16* xr = x + (size_t)r * ldx;
  float ss = 0.f;
  for (int c = threadIdx.x; c < hidden; c += 256) {
    float v = to_f32<DT>(xr[c]);
    ss += v * v;
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = (red[0] + red[1]) + (red[2] + red[3]);
  float inv = 1.0f / sqrtf(tot / (float)hidden + eps);
  u16* yr = y + (size_t)r * ldy;
  for (int c = threadIdx.x; c < hidden; c += 256) {
    float n = rnd<DT>(to_f32<DT>(xr[c]) * inv);
    yr[c] = from_f32<DT>(to_f32<DT>(w[c]) * n);
  }
}

// RoPE at absolute positions pos_offset + r (cuda.py:278-316) for q and k, then the in-place KV-cache
// append of k and v at rows [write_start, write_start + rows) (runtime.py:51-60).
template <int DT>
__global__ __launch_bounds__(256) void rope_kv_kernel(RopeArgs a) {
  const int r = blockIdx.x;
  const int half = a.hd / 2;
  const float pos = (float)r + (float)(*a.pos_offset);
  const u16* row = a.qkv + (size_t)r * a.ld;
  const int nrot = (a.nq + a.nkv) * half;
  const size_t crow = (size_t)(a.write_start + r) * a.nkv * a.hd;
  for (int t = threadIdx.x; t < nrot; t += 256) {
    const int head = t / half, i = t - head * half;
    float e = (a.neg_log_theta * (float)i) / (float)half;
    float inv_freq = expf(e);
    float fr = pos * inv_freq;
    float c = rnd<DT>(cosf(fr));
    float s = rnd<DT>(sinf(fr));
    const u16* src = row + head * a.hd;  // q heads, then k heads (contiguous in the qkv row)
    float x1 = to_f32<DT>(src[i]), x2 = to_f32<DT>(src[i + half]);
    u16 o1 = from_f32<DT>(rnd<DT>(x1 * c) + rnd<DT>(-x2 * s));
    u16 o2 = from_f32<DT>(rnd<DT>(x2 * c) + rnd<DT>(x1 * s));
    if (head < a.nq) {
      u16* dst = a.q_out + (size_t)r * a.nq * a.hd + head * a.hd;
      dst[i] = o1;
      dst[i + half] = o2;
    } else {
      u16* dst = a.k_cache + crow + (head - a.nq) * a.hd;
      dst[i] = o1;
      dst[i + half] = o2;
    }
  }
  const u16* vsrc = row + (a.nq + a.nkv) * a.hd;
  for (int t = threadIdx.x; t < a.nkv * a.hd; t += 256) a.v_cache[crow + t] = vsrc[t];
}

hipError_t launch_embed(const int32_t* ids, int n, const uint16_t* table, int vocab, int hidden, uint16_t* out,
                        hipStream_t st) {
  hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(256), 0, st, ids, table, vocab, hidden, out);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(int dt, const uint16_t* x, int ldx, int rows, int hidden, const uint16_t* w, float eps,
                          uint16_t* y, int ldy, hipStream_t st) {
  if (dt == DT_BF16)
    hipLaunchKernelGGL(rmsnorm_kernel<DT_BF16>, dim3(rows), dim3(256), 0, st, x, ldx, hidden, w, eps, y, ldy);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<DT_F16>, dim3(rows), dim3(256), 0, st, x, ldx, hidden, w, eps, y, ldy);
  return hipGetLastError();
}

hipError_t launch_rope_kv(int dt, const RopeArgs& a, hipStream_t st) {
  if (dt == DT_BF16)
    hipLaunchKernelGGL(rope_kv_kernel<DT_BF16>, dim3(a.rows), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(rope_kv_kernel<DT_F16>, dim3(a.rows), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace fdllm
