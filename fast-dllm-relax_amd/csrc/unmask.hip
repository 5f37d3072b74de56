// The threshold unmask of the decode loop on the device (fast_dllm_relax/runtime.py:794-805), alone or
// fused with the confidence combine of the lm_head's tile statistics, so that a decode step ends with
// the block's ids updated in device memory and a small report for the host (confidence.hpp).
#include "confidence.hpp"
#include "kernels.hpp"

namespace fdllm {

constexpr int UNMASK_MAX_ROWS = 1024;  // confidence rows one fused launch combines
constexpr int CONF_NT = 10;            // tiles per lane held in registers (594 for the 1.5B vocabulary)

// One workgroup: its waves combine the rows' tile statistics (wave w takes rows w, w + nw, ...), then
// wave 0 applies the rule to the sub-block.
__global__ __launch_bounds__(1024) void confidence_unmask_kernel(const float* stat_m, const int32_t* stat_a,
                                                                 const float* stat_s, int tiles,
                                                                 int32_t* ids_out, float* maxp_out, UnmaskP u) {
  __shared__ int32_t ids_l[UNMASK_MAX_ROWS];
  __shared__ float maxp_l[UNMASK_MAX_ROWS];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  auto put = [&](int r, int32_t id, float p) {
    if (lane == 0) {
      ids_l[r] = id;
      maxp_l[r] = p;
      if (ids_out != nullptr) {
        ids_out[r] = id;
        maxp_out[r] = p;
      }
    }
  };
  if (tiles <= 64 * CONF_NT && u.rows <= 2 * nw) {
    // a decode step's rows (up to 32 on 16 waves): rows w and w + nw together, every statistic in one
    // round trip (about 10 us -> 4 us for 32 rows of the 1.5B vocabulary)
    int32_t id[2];
    float p[2];
    const int nr = (w < u.rows ? 1 : 0) + (w + nw < u.rows ? 1 : 0);  // rows w and w + nw
    confidence_rows<2, CONF_NT>(stat_m + (size_t)w * tiles, stat_a + (size_t)w * tiles, stat_s + (size_t)w * tiles,
                                tiles, nw * tiles, nr, lane, id, p);
    if (nr > 0) put(w, id[0], p[0]);
    if (nr > 1) put(w + nw, id[1], p[1]);
  } else {
    for (int r = w; r < u.rows; r += nw) {
      int32_t id;
      float p;
      confidence_row(stat_m + (size_t)r * tiles, stat_a + (size_t)r * tiles, stat_s + (size_t)r * tiles, tiles, lane,
                     &id, &p);
      put(r, id, p);
    }
  }
  __syncthreads();
  if (w == 0) unmask_wave(ids_l, maxp_l, u, lane);
}

// The rule alone, on a confidence the caller holds (fdllm_get_confidence's outputs).
__global__ __launch_bounds__(64) void unmask_kernel(const int32_t* ids, const float* maxp, UnmaskP u) {
  unmask_wave(ids, maxp, u, threadIdx.x);
}

hipError_t launch_confidence_unmask(const float* sm, const int32_t* sa, const float* ss, int tiles, int stat_rows,
                                    int32_t* ids, float* maxp, const UnmaskP& u, hipStream_t st) {
  if (u.rows <= 0 || u.rows > UNMASK_MAX_ROWS || u.rows > stat_rows) return hipErrorInvalidValue;
  const int nw = u.rows < 16 ? u.rows : 16;
  hipLaunchKernelGGL(confidence_unmask_kernel, dim3(1), dim3(64 * nw), 0, st, sm, sa, ss, tiles, ids, maxp, u);
  return hipGetLastError();
}

hipError_t launch_unmask(const int32_t* ids, const float* maxp, const UnmaskP& u, hipStream_t st) {
  hipLaunchKernelGGL(unmask_kernel, dim3(1), dim3(64), 0, st, ids, maxp, u);
  return hipGetLastError();
}

}  // namespace fdllm
