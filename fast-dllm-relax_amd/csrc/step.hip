// Planning and launch of the persistent cached-step kernel (step_body.hpp).
#include "step_body.hpp"

#include <algorithm>

namespace fdllm {

__global__ __launch_bounds__(256) void fill_u32_kernel(unsigned* p, size_t n, unsigned v) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = v;
}

hipError_t launch_fill_u32(unsigned* p, size_t n, unsigned v, hipStream_t st) {
  const int blocks = (int)std::min<size_t>(64, (n + 255) / 256);
  hipLaunchKernelGGL(fill_u32_kernel, dim3(std::max(blocks, 1)), dim3(256), 0, st, p, n, v);
  return hipGetLastError();
}

size_t step_sync_words(const StepP& p) {
  return (size_t)BAR_CTRS * BAR_STRIDE + (size_t)std::max(p.d_groups, 1) * BAR_STRIDE + BAR_STRIDE;
}

// LDS of the attention chunk body (attn_chunk_compute with 4 query tiles x 2 key parts: K, V^T and the
// query fragments)
static size_t chunk_lds(int ch) {
  const size_t loop = (size_t)ch * KLD * 2 + (size_t)HD * (ch + 8) * 2 + (size_t)4 * 4 * 64 * 16;
  const size_t merge = (size_t)2 * 2 * 4 * 16 * 4 + (size_t)1 * 4 * (HD / 16) * 64 * 16;
  return std::max(loop, merge);
}

StepPlan step_plan(const StepP& p, int G) {
  StepPlan r{false, nullptr, 0};
  const int KSH = p.H / 32, KSO = p.q_dim / 32, KSD = p.I / 32;
  const int grp = p.nq / p.nkv, QT = (grp * p.M + 15) / 16;
  if (p.M < 1 || p.M > 32) { r.why = "more than 32 rows"; return r; }
  if (p.H % 32 || p.q_dim % 32 || p.I % 32) { r.why = "dimensions not multiples of 32"; return r; }
  if (KSH > 8 * STEP_KPW || KSO > 8 * STEP_KPW) { r.why = "hidden or q width above 1536"; return r; }
  if (p.nt_q > G || p.nt_o > G || p.np_u > STEP_PAIRS * G) { r.why = "projection wider than the grid"; return r; }
  if (p.d_splits < 1 || KSD % p.d_splits || KSD / p.d_splits > 8 * STEP_DKPW || p.d_groups * p.d_splits > G) {
    r.why = "down split does not fit";
    return r;
  }
  if (p.at.chunk != 64 && p.at.chunk != 128) { r.why = "attention chunk"; return r; }
  if (QT > 4 * p.qg || p.qg * p.nkv * p.at.S > G || 8 * QT * p.nkv > 8 * G) { r.why = "attention wider than the grid"; return r; }
  size_t lds = STEP_LDS;  // weight slices and wave sums (step_body.hpp)
  lds = std::max(lds, (size_t)8 * STEP_DKPW * STEP_DNT * 1024);
  lds = std::max(lds, chunk_lds(p.at.chunk));
  if (lds > 160 * 1024) { r.why = "LDS"; return r; }
  r.ok = true;
  r.lds = lds;
  return r;
}

template <int DT, int CH>
static hipError_t launch_ch(const StepP& p, int G, size_t lds, hipStream_t st) {
  auto kern = step_kernel<DT, CH>;
  static size_t attr_lds = 0;  // per instantiation
  if (lds > 64 * 1024 && lds > attr_lds) {
    const hipError_t e =
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_lds = lds;
  }
  StepP arg = p;
  void* args[] = {&arg};
  return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kern), dim3(G), dim3(512), args, (unsigned)lds, st);
}

template <int DT>
static hipError_t launch_dt(const StepP& p, int G, size_t lds, hipStream_t st) {
  if (p.at.chunk == 64) return launch_ch<DT, 64>(p, G, lds, st);
  return launch_ch<DT, 128>(p, G, lds, st);
}

hipError_t launch_step(int dt, const StepP& p, int G, size_t lds, hipStream_t st) {
  if (dt == DT_BF16) return launch_dt<DT_BF16>(p, G, lds, st);
  return launch_dt<DT_F16>(p, G, lds, st);
}

}  // namespace fdllm
