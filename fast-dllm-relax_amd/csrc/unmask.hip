// The threshold unmask of the decode loop on the device (fast_dllm_relax/runtime.py:794-805), alone or
// fused with the confidence combine of the lm_head's tile statistics, so that a decode step ends with
// the block's ids updated in device memory and a small report for the host (confidence.hpp).
#include "confidence.hpp"
#include "kernels.hpp"

namespace fdllm {

constexpr int UNMASK_MAX_ROWS = 1024;  // confidence rows one fused launch combines
constexpr int CONF_NT = 10;            // tiles per lane held in registers (594 for the 1.5B vocabulary)

// One workgroup: its waves combine the rows' tile statistics, then wave 0 applies the rule to the
// sub-block.  The rule reads the confidence of rows row0 - 1 .. row0 + sub - 1 (the shift) and, for the
// report, of the last row; unless the caller asks for every row's confidence (ids_out), only those
// (up to sub + 2 of them) are combined: a decode step's 9 or 10 of 32 rows.  A row's statistics are
// read by one compute unit, so the rows it skips are the kernel's time: 13.5 -> 8.0 us per decode call
// when each wave first requested both of its rows together, 8.0 -> 6.2 us with 9 or 10 rows instead of
// 32 (the rest is the launch, the first-touch latency of the statistics and the report's system fence).
struct UnmaskRows {
  int all;     // every row [0, rows)
  int lo, n;   // else rows lo .. lo + n - 1 (and, when extra, the last row as the n-th)
  int extra;
};
__host__ __device__ inline UnmaskRows unmask_rows(const UnmaskP& u, bool all) {
  UnmaskRows r{};
  r.all = all;
  if (all) return r;
  if (u.sub == 0) {  // no update: the report's last-row prediction only
    r.extra = u.report != nullptr ? 1 : 0;
    return r;
  }
  r.lo = u.row0 > 0 ? u.row0 - 1 : 0;
  const int hi = u.row0 + u.sub - 1;
  r.n = hi - r.lo + 1;
  r.extra = u.report != nullptr && u.rows - 1 > hi ? 1 : 0;
  return r;
}

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
  const UnmaskRows sel = unmask_rows(u, ids_out != nullptr);
  if (!sel.all) {
    // the rows the rule reads, one per wave while they last
    for (int k = w; k < sel.n + sel.extra; k += nw) {
      const int r = k < sel.n ? sel.lo + k : u.rows - 1;
      int32_t id;
      float p;
      if (tiles <= 64 * CONF_NT)
        confidence_rows<1, CONF_NT>(stat_m + (size_t)r * tiles, stat_a + (size_t)r * tiles, stat_s + (size_t)r * tiles,
                                    tiles, tiles, 1, lane, &id, &p);
      else
        confidence_row(stat_m + (size_t)r * tiles, stat_a + (size_t)r * tiles, stat_s + (size_t)r * tiles, tiles, lane,
                       &id, &p);
      put(r, id, p);
    }
  } else if (tiles <= 64 * CONF_NT && u.rows <= 2 * nw) {
    // every row (up to 32 on 16 waves): rows w and w + nw together, every statistic in one round trip
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
  const UnmaskRows sel = unmask_rows(u, ids != nullptr);
  const int want = sel.all ? u.rows : sel.n + sel.extra;
  const int nw = want < 1 ? 1 : want < 16 ? want : 16;
  hipLaunchKernelGGL(confidence_unmask_kernel, dim3(1), dim3(64 * nw), 0, st, sm, sa, ss, tiles, ids, maxp, u);
  return hipGetLastError();
}

hipError_t launch_unmask(const int32_t* ids, const float* maxp, const UnmaskP& u, hipStream_t st) {
  hipLaunchKernelGGL(unmask_kernel, dim3(1), dim3(64), 0, st, ids, maxp, u);
  return hipGetLastError();
}

}  // namespace fdllm
