// GQA attention of the block rows against the in-place KV cache (fast_dllm.attn_inplace,
// fast_dllm_relax/runtime.py:63-73; in-graph restatement model/metal.py:378-408): query head h uses
// kv head h / (nq / nkv); scores q.k * scale in fp32, softmax in fp32, P.V with fp32 accumulation.
//
// Work split: blockIdx.y = kv head, blockIdx.z = key split, blockIdx.x = group of 4 query tiles.
// The group's query rows of all heads sharing the kv head are stacked (row qi = head_in_group * R + r),
// so one K/V stream serves all of them.  Each wave owns 16 query rows:
//   S^T = K . Q^T   (A = 16 keys x 32 dims straight from the cache rows, B = the wave's queries)
// leaves lane l with 4 keys of query l % 16, which is exactly the A-operand layout P needs for
//   O = P . V       (B = V^T from LDS, keys permuted consistently with P's register order).
// Online softmax inside a split; the splits are merged by attn_combine_kernel.
#include "common.hpp"
#include "kernels.hpp"

namespace fdllm {

constexpr int HD = 128;
constexpr int KSUB = 64;      // keys per inner step
constexpr int VT_LD = KSUB + 8;

template <int DT>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
  __shared__ __align__(16) u16 vt[HD * VT_LD];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int g = blockIdx.y, split = blockIdx.z;
  const int grp = a.nq / a.nkv;
  const int QR = grp * a.rows;
  const int qt = blockIdx.x * 4 + w;
  const bool active = qt * 16 < QR;
  const size_t krow = (size_t)a.nkv * HD;

  const int qi = qt * 16 + lr;
  const bool qvalid = qi < QR;
  const int hh = qvalid ? qi / a.rows : 0;
  const int r = qvalid ? qi - hh * a.rows : 0;
  u32x4 qf[HD / 32];
  {
    const u16* qp = a.q + (size_t)r * a.nq * HD + (g * grp + hh) * HD + 8 * lg;
#pragma unroll
    for (int ds = 0; ds < HD / 32; ++ds)
      qf[ds] = qvalid ? *reinterpret_cast<const u32x4*>(qp + 32 * ds) : u32x4{0u, 0u, 0u, 0u};
  }
  const int qpos_blk = (a.q_pos0 + r) / (a.block > 0 ? a.block : 1);
  const float* brow = a.mask == 2 ? a.bias + (long long)r * a.bias_ld : nullptr;

  const int kbeg = split * a.chunk;
  const int kend = min(kbeg + a.chunk, a.Lk);

  float m_run = -INFINITY, l_run = 0.f;
  f32x4 o[HD / 16];
#pragma unroll
  for (int dt = 0; dt < HD / 16; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int kb = kbeg; kb < kend; kb += KSUB) {
    __syncthreads();
    for (int idx = threadIdx.x; idx < KSUB * (HD / 8); idx += 256) {
      const int key = idx % KSUB, dblk = idx / KSUB;
      const int kk = kb + key;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (kk < kend) val = *reinterpret_cast<const u32x4*>(a.v + kk * krow + g * HD + dblk * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) vt[(dblk * 8 + e) * VT_LD + key] = (u16)(val[e >> 1] >> (16 * (e & 1)));
    }
    __syncthreads();
    if (!active) continue;

    f32x4 s[KSUB / 16];
#pragma unroll
    for (int kt = 0; kt < KSUB / 16; ++kt) {
      s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
      int key = kb + 16 * kt + lr;
      key = key < kend ? key : kend - 1;
      const u16* kp = a.k + key * krow + g * HD + 8 * lg;
#pragma unroll
      for (int ds = 0; ds < HD / 32; ++ds)
        s[kt] = mfma16<DT>(*reinterpret_cast<const u32x4*>(kp + 32 * ds), qf[ds], s[kt]);
    }
    // lane holds S^T[key = kb + 16 kt + 4 lg + i][query lr]
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < KSUB / 16; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kb + 16 * kt + 4 * lg + i;
        float v = s[kt][i] * a.scale;
        if (key >= kend) {
          v = -INFINITY;
        } else if (a.mask == 1) {
          if (qpos_blk < key / a.block) v = -INFINITY;
        } else if (a.mask == 2) {
          v += brow[key];
        }
        s[kt][i] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, WAVE));
    mx = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = expf(m_run - m_use);
    float ps = 0.f;
#pragma unroll
    for (int kt = 0; kt < KSUB / 16; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float p = expf(s[kt][i] - m_use);
        s[kt][i] = p;
        ps += p;
      }
    ps += __shfl_xor(ps, 16, WAVE);
    ps += __shfl_xor(ps, 32, WAVE);
    l_run = l_run * alpha + ps;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float al = __shfl(alpha, 4 * lg + i, WAVE);
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt) o[dt][i] *= al;
    }
#pragma unroll
    for (int ks = 0; ks < KSUB / 32; ++ks) {
      u16 pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = from_f32<DT>(s[2 * ks + (e >> 2)][e & 3]);
      u32x4 pa = {(uint32_t)pv[0] | ((uint32_t)pv[1] << 16), (uint32_t)pv[2] | ((uint32_t)pv[3] << 16),
                  (uint32_t)pv[4] | ((uint32_t)pv[5] << 16), (uint32_t)pv[6] | ((uint32_t)pv[7] << 16)};
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt) {
        const u16* vrow = vt + (16 * dt + lr) * VT_LD + 32 * ks + 4 * lg;
        u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
        u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 16);
        u32x4 vb = {lo[0], lo[1], hi[0], hi[1]};
        o[dt] = mfma16<DT>(pa, vb, o[dt]);
      }
    }
  }
  if (!active) return;
  const size_t base = (size_t)(split * a.nkv + g) * a.QRp;
#pragma unroll
  for (int dt = 0; dt < HD / 16; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) a.o_part[(base + qt * 16 + 4 * lg + i) * HD + 16 * dt + lr] = o[dt][i];
  if (lg == 0) {
    a.m_part[base + qt * 16 + lr] = m_run;
    a.l_part[base + qt * 16 + lr] = l_run;
  }
}

// Merge the key splits: out = sum_s exp(m_s - M) O_s / sum_s exp(m_s - M) l_s, cast once.
template <int DT>
__global__ __launch_bounds__(128) void attn_combine_kernel(AttnArgs a) {
  const int r = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const int grp = a.nq / a.nkv;
  const int g = h / grp, hh = h - g * grp;
  const int qi = hh * a.rows + r;
  float M = -INFINITY;
  for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, a.m_part[(size_t)(s * a.nkv + g) * a.QRp + qi]);
  const float Mu = M == -INFINITY ? 0.f : M;
  float L = 0.f, acc = 0.f;
  for (int s = 0; s < a.nsplit; ++s) {
    const size_t b = (size_t)(s * a.nkv + g) * a.QRp + qi;
    const float wgt = expf(a.m_part[b] - Mu);
    L += a.l_part[b] * wgt;
    acc += a.o_part[b * HD + d] * wgt;
  }
  a.out[(size_t)r * a.nq * HD + h * HD + d] = from_f32<DT>(acc / L);
}

hipError_t launch_attention(int dt, const AttnArgs& a, int nqgroups, hipStream_t st) {
  if (a.hd != HD) return hipErrorInvalidValue;
  if (dt == DT_BF16) {
    hipLaunchKernelGGL(attn_kernel<DT_BF16>, dim3(nqgroups, a.nkv, a.nsplit), dim3(256), 0, st, a);
    hipLaunchKernelGGL(attn_combine_kernel<DT_BF16>, dim3(a.rows, a.nq), dim3(HD), 0, st, a);
  } else {
    hipLaunchKernelGGL(attn_kernel<DT_F16>, dim3(nqgroups, a.nkv, a.nsplit), dim3(256), 0, st, a);
    hipLaunchKernelGGL(attn_combine_kernel<DT_F16>, dim3(a.rows, a.nq), dim3(HD), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace fdllm
