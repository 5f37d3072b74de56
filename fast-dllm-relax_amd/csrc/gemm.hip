// Skinny GEMM launch planning and launchers, the confidence kernels and the weight repack; the GEMM
// kernels and their bodies are in gemm_body.hpp.
#include "confidence.hpp"
#include "gemm_body.hpp"
#include "gemm_mm.hpp"
#include "gemm_wt.hpp"

#include <algorithm>

namespace fdllm {

// One wave per row: combine the tile statistics into (argmax, maxp) in the fixed lane order.
__global__ __launch_bounds__(64) void confidence_combine_kernel(const float* stat_m, const int32_t* stat_a,
                                                                const float* stat_s, int tiles, int rows,
                                                                int32_t* ids, float* maxp) {
  const int r = blockIdx.x, lane = threadIdx.x;
  if (r >= rows) return;
  int32_t id;
  float p;
  if (tiles <= 64 * 10) {
    // the row's statistics requested together: one memory round trip (the 1.5B vocabulary's 594 tiles)
    confidence_rows<1, 10>(stat_m + (size_t)r * tiles, stat_a + (size_t)r * tiles, stat_s + (size_t)r * tiles, tiles,
                           tiles, 1, lane, &id, &p);
  } else {
    confidence_row(stat_m + (size_t)r * tiles, stat_a + (size_t)r * tiles, stat_s + (size_t)r * tiles, tiles, lane,
                   &id, &p);
  }
  if (lane == 0) {
    ids[r] = id;
    maxp[r] = p;
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
    const int c = n0 + lane + 64 * i;
    if (c < vocab) {
      const float x = row[c];
      if (x > vmax) { vmax = x; amax = c; }
    }
  }
  for (int k = 32; k >= 1; k >>= 1) {
    const float ov = __shfl_xor(vmax, k, WAVE);
    const int oa = __shfl_xor(amax, k, WAVE);
    if (ov > vmax || (ov == vmax && oa < amax)) { vmax = ov; amax = oa; }
  }
  float s = 0.0f;
  for (int i = 0; i < 4; ++i) {
    const int c = n0 + lane + 64 * i;
    if (c < vocab) s = s + fd_exp_neg(row[c] - vmax);
  }
  for (int k = 32; k >= 1; k >>= 1) s = s + __shfl_xor(s, k, WAVE);
  if (lane == 0) {
    const size_t o = (size_t)r * tiles + t;
    stat_m[o] = vmax;
    stat_a[o] = amax;
    stat_s[o] = s;
  }
}

// Weight repack into fragment order (one thread per 16-byte output chunk).
__global__ __launch_bounds__(256) void pack_kernel(const u16* src, int N, int K, size_t total, int mode, u16* dst) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int KS = K / 32;
  const int l = (int)(idx & 63);
  const size_t ts = idx >> 6;
  const int s = (int)(ts % KS);
  const int t = (int)(ts / KS);
  const int r = l & 15, g = l >> 4;
  int row;
  bool ok;
  if (mode == PACK_PAIRS) {
    const int half = N / 2;
    const int i = 16 * (t >> 1) + r;
    ok = i < half;
    row = (t & 1) ? half + i : i;
  } else {
    row = 16 * t + r;
    ok = row < N;
  }
  u32x4 v = {0u, 0u, 0u, 0u};
  if (ok) v = *reinterpret_cast<const u32x4*>(src + (size_t)row * K + 32 * s + 8 * g);
  *reinterpret_cast<u32x4*>(dst + idx * 8) = v;
}

// ---- launchers ---------------------------------------------------------------------------------
template <int EPI, int XF, int TPW, int TW, int KW, int U>
struct Cfg {
  static constexpr int epi = EPI, xf = XF, tpw = TPW, tw = TW, kw = KW, u = U;
};
// streaming kernel (any M: prefill chunks, the lm_head)
using CfgQkv = Cfg<EPI_BIAS, XF_RMS, 1, 1, 8, 3>;
using CfgOproj = Cfg<EPI_RESID, XF_NONE, 1, 1, 8, 3>;
using CfgGateUp = Cfg<EPI_SILU_PAIR, XF_RMS, 2, 2, 2, 4>;
using CfgDown = Cfg<EPI_RESID, XF_NONE, 1, 4, 2, 4>;
using CfgLmHead = Cfg<EPI_LOGITS, XF_NONE, 4, 4, 1, 2>;
// one-shot kernel (M <= 32): tiles per workgroup, max k steps per wave, preferred k split
template <int EPI, int XF, int NT, int KPW, int SPLIT>
struct OsCfg {
  static constexpr int epi = EPI, xf = XF, nt = NT, kpw = KPW, split = SPLIT;
};
using OsQkv = OsCfg<EPI_BIAS, XF_RMS, OsQkvNT, OsQkvKPW, OsQkvSplit>;
using OsOproj = OsCfg<EPI_RESID, XF_NONE, OsOprojNT, OsOprojKPW, OsOprojSplit>;
using OsGateUp = OsCfg<EPI_SILU_PAIR, XF_RMS, OsGateUpNT, OsGateUpKPW, OsGateUpSplit>;
using OsDown = OsCfg<EPI_RESID, XF_NONE, OsDownNT, OsDownKPW, OsDownSplit>;
using OsNone = OsCfg<EPI_LOGITS, XF_NONE, 0, 0, 1>;

template <class C> constexpr int tiles_of() { return C::tpw * C::tw; }

static int streaming_tiles(int cfg) {
  switch (cfg) {
    case CFG_QKV: return tiles_of<CfgQkv>();
    case CFG_OPROJ: return tiles_of<CfgOproj>();
    case CFG_GATE_UP: return tiles_of<CfgGateUp>();
    case CFG_DOWN: return tiles_of<CfgDown>();
    default: return tiles_of<CfgLmHead>();
  }
}
struct OsInfo { int nt, kpw, split; };
static OsInfo os_info(int cfg) {
  switch (cfg) {
    case CFG_QKV: return {OsQkv::nt, OsQkv::kpw, OsQkv::split};
    case CFG_OPROJ: return {OsOproj::nt, OsOproj::kpw, OsOproj::split};
    case CFG_GATE_UP: return {OsGateUp::nt, OsGateUp::kpw, OsGateUp::split};
    case CFG_DOWN: return {OsDown::nt, OsDown::kpw, OsDown::split};
    default: return {0, 0, 1};
  }
}

GemmShape gemm_shape(int cfg) {
  const int a = streaming_tiles(cfg), b = os_info(cfg).nt;
  int l = a;
  if (b > 0) {
    int x = a, y = b;
    while (y != 0) { const int r = x % y; x = y; y = r; }
    l = a / x * b;
  }
  return GemmShape{l, 0};
}

// rows from which the lm_head (with its confidence statistics) takes the register-weight kernel (us per
// launch with the statistics, fp16, register-weight / 64 x 256 LDS-staged blocks: 199 / 228-232 at 256 rows,
// 326 / 386 at 512, even at 112-128)
#ifndef FD_WR_LM_MIN_ROWS
#define FD_WR_LM_MIN_ROWS 256
#endif
// stages in flight of the register-weight kernel
#ifndef FD_WR_DEPTH
#define FD_WR_DEPTH 3
#endif

// large-M kernel configurations (rows x columns per workgroup)
using MmSmall = MmCfg<4, 2, 1, 4, 2, 2>;  // 64 x 128, weights two stages ahead
using MmWide = MmCfg<4, 4, 1, 4, 2, 1>;   // 64 x 256
using MmWideD = MmCfg<4, 4, 1, 4, 2, 2>;  // 64 x 256, weights two stages ahead
using MmBig = MmCfg<8, 2, 1, 8, 2, 1>;    // 128 x 256, 8 waves
// LDS-staged kernel (gemm_wt.hpp): 2 x 2 waves of 64 x 96, a 128 x 192 block, four stage buffers of
// 20 KB (two workgroups per compute unit)
template <int MF, int TPW, int WM, int WN, int NBUF>
struct WtCfg {
  static constexpr int mf = MF, tpw = TPW, wm = WM, wn = WN, nw = WM * WN, nbuf = NBUF;
  static constexpr int bm = 16 * MF * WM, bn_tiles = TPW * WN, kss = 1;
  static constexpr size_t lds = (size_t)NBUF * (MF * WM + TPW * WN) * 1024;
};
using WtBig = WtCfg<4, 6, 2, 2, 4>;
// 4 x 2 waves of 32 x 96 (124 registers, two workgroups and 16 waves per compute unit; waves copy 3 or 2
// of the 20 blocks a stage).  gate_up, us per launch with its norm pass, eight / four waves: 43.4 / 43.8 at
// 384 rows, 44.4 / 44.7 at 512, 58.8 / 59.6 at 768, 60.6 / 61.4 at 1024; down unchanged (28.6 at 512)
using WtBig8 = WtCfg<2, 6, 4, 2, 4>;
// 4 x 2 waves of 64 x 96: a 256 x 192 block, one workgroup per compute unit (189 registers, 112 KB of LDS;
// waves copy 4 or 3 of a stage's 28 blocks), 30% less data into the compute units than the 128 x 192
// blocks.  gate_up with its norm pass: 42.5 against 44.3 us at 512 rows (188 workgroups), 41.9 against
// 43.4 at 384; with four waves of 128 x 96 the same block took 67 against 46
using WtB256 = WtCfg<4, 6, 4, 2, 4>;
// register-weight kernel (gemm_wt.hpp, gemm_wr_kernel): four waves of 16 MF rows x TPW tiles, a
// 16 MF x 64 TPW block, D stages in flight
template <int MF, int TPW, int D>
struct WrCfg {
  static constexpr int mf = MF, tpw = TPW, d = D;
  static constexpr int bm = 16 * MF, bn_tiles = 4 * TPW, kss = 1;
  static constexpr size_t lds = (size_t)(D + 1) * MF * 1024;
  static constexpr size_t lds_logits = (size_t)16 * MF * 256 * 2;  // the lm_head's [BM][256] logit tile
};
using WrBig = WrCfg<8, 4, FD_WR_DEPTH>;  // 128 x 256
// stages in flight of the small register-weight blocks (8 MFMAs per k step and wave cover little latency)
#ifndef FD_WR_SMALL_DEPTH
#define FD_WR_SMALL_DEPTH 8
#endif
using WrSmall = WrCfg<4, 2, FD_WR_SMALL_DEPTH>;  // 64 x 128
using WrMid = WrCfg<8, 2, 6>;    // 128 x 128 (six stages: 56 KB of LDS)
using WrTiny = WrCfg<4, 1, 12>;  // 64 x 64 (4 MFMAs per k step and wave: twelve stages in flight)
// (qkv with RoPE in the epilogue exchanges rotation partners between waves through the stage buffers)
static_assert(WrTiny::lds >= (size_t)4 * 1 * 4 * 64 * 8 && WrSmall::lds >= (size_t)4 * 2 * 4 * 64 * 8,
              "the RoPE exchange fits the stage buffers");
// 128 x 192 (o_proj / down from the register-weight thresholds: 1536 columns make 8 column blocks, so
// 64 row blocks of 8192 rows fill 512 slots, two per compute unit, where the 128 x 256 blocks' 384
// leave half the units with one)
using WrB3 = WrCfg<8, 3, FD_WR_DEPTH>;
enum MmId : int { MM_SMALL = 0, MM_WIDE = 1, MM_WIDE_D = 2, MM_BIG = 3, MM_WT = 4, MM_WR = 5, MM_WR_S = 6, MM_WR_M = 7, MM_WR_T = 8, MM_WR_3 = 9, MM_WT_8 = 10, MM_WT_256 = 11 };
struct MmInfo { int bm, bn_tiles, kss; };
template <class M> constexpr MmInfo mm_info_of() { return MmInfo{M::bm, M::bn_tiles, M::kss}; }
static MmInfo mm_info(int id) {
  switch (id) {
    case MM_WIDE: return mm_info_of<MmWide>();
    case MM_WIDE_D: return mm_info_of<MmWideD>();
    case MM_BIG: return mm_info_of<MmBig>();
    case MM_WT: return mm_info_of<WtBig>();
    case MM_WR: return mm_info_of<WrBig>();
    case MM_WR_S: return mm_info_of<WrSmall>();
    case MM_WR_M: return mm_info_of<WrMid>();
    case MM_WR_T: return mm_info_of<WrTiny>();
    case MM_WR_3: return mm_info_of<WrB3>();
    case MM_WT_8: return mm_info_of<WtBig8>();
    case MM_WT_256: return mm_info_of<WtB256>();
    default: return mm_info_of<MmSmall>();
  }
}
// Rows from which a projection takes the register-weight kernel by default.  Measured (1.5B, us per
// launch, register-weight / previous kernel): gate_up 53 / 47 at 512 rows, 110 / 118 at 2048, 377 / 448
// at 8192; down 40 / 30, 79 / 80, 189 / 192; qkv 37 / 31 at 2048, 75 / 106 at 8192; o_proj 38 / 23,
// 57 / 70.  Below these sizes its 128 x 256 blocks leave too few workgroups without a k split.
static int wr_default_min_rows(int cfg) {
  if (cfg == CFG_LM_HEAD) return FD_WR_LM_MIN_ROWS;
  return cfg == CFG_GATE_UP || cfg == CFG_DOWN ? 2048 : 4096;
}
static int mm_choice(int cfg, int M, int ntiles, const MmPolicy& pol) {
  const int min_rows = pol.wr_min_rows > 0 ? pol.wr_min_rows : wr_default_min_rows(cfg);
  if (M >= std::max(min_rows, 33) && ((pol.wr_ops >> cfg) & 1))
    return pol.wr3 && (cfg == CFG_OPROJ || cfg == CFG_DOWN) && ntiles % WrB3::bn_tiles == 0 ? MM_WR_3 : MM_WR;
  // qkv and o_proj below that: 64 x 128 register-weight blocks (us per launch, qkv including its norm pass,
  // against the LDS-staged 64 x 128 kernel): qkv 16.2 / 14.9 at 128 rows, 23.2 / 20.2 at 512, 26.2 / 19.4
  // at 1024, 30.8 / 28.6 at 2048; o_proj 15.2 / 14.0 at 384, 15.4 / 14.0 at 512, 19.3 / 15.1 at 1024, but
  // 23.3 / 26.4 at 2048 (equal below 384).  Up to 512 rows 64 x 64 blocks, twice the workgroups, do better
  // still (us, 64 x 128 / 64 x 64 blocks): qkv 14.4 / 13.4 at 128 rows, 15.7 / 13.7 at 256, 16.8 / 14.9 at
  // 512 (but 19.4 / 21.2 at 1024); o_proj 12.8 / 11.9, 12.8 / 11.9, 14.0 / 12.0 (15.1 / 21.4 at 1024)
  if (M >= 33 && ((pol.wr_small_ops >> cfg) & 1) && (cfg == CFG_QKV || (cfg == CFG_OPROJ && M < 2048)))
    return M <= 512 ? MM_WR_T : MM_WR_S;
  // gate_up and down below 256 rows: register-weight blocks too (us per launch, gate_up including its norm
  // pass; LDS-staged kernel / 64 x 128 / 128 x 128 blocks): gate_up 24.8 / 21.3 / 22.7 at 64 rows, 30.0 /
  // 29.9 / 26.1 at 128, 38.6 / 29.5 / 35.6 at 192; down 21.4 / 16.8 / 18.0, 21.4 / 18.0 / 20.8, 27.1 / 24.7 /
  // 25.2.  The 128 x 128 blocks win where they make one round of workgroups and the 64 x 128 ones two.
  if (M >= 33 && M < 256 && (cfg == CFG_GATE_UP || cfg == CFG_DOWN)) {
    const int sh = cfg == CFG_GATE_UP ? 0 : 1;
    const int ffn = pol.wr_ffn >= 0 ? pol.wr_ffn : (M > 64 && M <= 128 ? 4 | 2 : 1 | 2);
    if ((ffn >> sh) & 1) return MM_WR_S;
    if ((ffn >> (sh + 2)) & 1) return MM_WR_M;
  }
  switch (cfg) {
    case CFG_LM_HEAD: return MM_WIDE;  // one 256-column confidence tile per block column
    case CFG_GATE_UP:
      if (M > 256 && M <= pol.wt256 && ntiles % WtB256::bn_tiles == 0) return MM_WT_256;
      if (M >= 256 && ntiles % WtBig::bn_tiles == 0) return (pol.wt8 & 1) ? MM_WT_8 : MM_WT;
      return M >= 1024 ? MM_BIG : MM_WIDE;
    case CFG_DOWN:
      if (M >= 256 && ntiles % WtBig::bn_tiles == 0) return (pol.wt8 & 2) ? MM_WT_8 : MM_WT;
      return M >= 1024 ? MM_WIDE_D : MM_SMALL;
    default:  // qkv, o_proj: the LDS-staged kernel measured slower at their widths (2048 / 1536 columns)
      return MM_SMALL;
  }
}

GemmPlan gemm_plan(int cfg, GemmP& a, int stream_split, const MmPolicy& pol) {
  GemmPlan p{};
  p.mchunks = (a.M + 31) / 32;
  if (a.M > 32) {
    const int id = mm_choice(cfg, a.M, a.ntiles, pol);
    const MmInfo mi = mm_info(id);
    if (a.KS % mi.kss == 0) {
      const int nst = a.KS / mi.kss;
      p.kind = GK_MM;
      p.mm_id = id;
      p.nbm = (a.M + mi.bm - 1) / mi.bm;
      p.nbn = (a.ntiles + mi.bn_tiles - 1) / mi.bn_tiles;
      // k split: the smallest divisor of the stage count that brings the launch to mm_target_wgs
      // workgroups (at most 8 splits of at least mm_min_stages stages), else the largest such divisor
      const int wgs = p.nbm * p.nbn;
      // (up to 128 rows, half the target: a split's fp32 partials and its epilogue launch cost more
      // than the idle compute units; measured on the 128-row batched step, 3.15 -> 2.93 ms)
      // o_proj (48 k steps) a quarter: at 512 rows its 96 workgroups without a split took 15.4 us against
      // 18.9 us split three ways with the epilogue launch
      int target = a.M <= 128 ? pol.target_wgs / 2 : pol.target_wgs;
      if (cfg == CFG_OPROJ) target /= 4;
      // qkv on the 64 x 128 (and 64 x 64) register-weight blocks half: 17.1 against 20.4 us at 512 rows (128 workgroups
      // without a split against 256 with one), 13.8 against 14.5 at 128 (two splits against four)
      if (cfg == CFG_QKV && (id == MM_WR_S || id == MM_WR_T)) target /= 2;
      // down above 128 rows seven eighths: at 512 rows seven splits (224 workgroups) against eight (256)
      // measured 3.92 against 3.94-3.95 ms per batched step (fewer partials for the split sum; five
      // splits 4.03, ten 3.95)
      if (cfg == CFG_DOWN && a.M > 128) target = target * 7 / 8;
      if (id == MM_WT_256) target = 0;  // no split
      int split = 1;
      const int max_split = id == MM_WR || id == MM_WR_S || id == MM_WR_M || id == MM_WR_T || id == MM_WR_3 ? 16 : 8;
      if (pol.force_split > 1 && cfg != CFG_LM_HEAD && nst % pol.force_split == 0 && nst / pol.force_split >= pol.min_stages)
        split = pol.force_split;
      else
        for (int d = 2; d <= max_split && wgs * split < target && cfg != CFG_LM_HEAD; ++d)
          if (nst % d == 0 && nst / d >= pol.min_stages) split = d;
      p.ksplit = split;
      a.kps = a.KS / split;
      p.part_floats = split > 1 ? (size_t)split * a.ntiles * ((a.M + 15) / 16) * 256 : 0;
      return p;
    }
  }
  const OsInfo o = os_info(cfg);
  // One-shot qkv and o_proj keep one weight tile per workgroup (128 / 96 workgroups at the 1.5B shapes),
  // so with 32 rows a compute unit takes in twice as many activation bytes (96 KB) as weight bytes.
  // Two 16-row m-chunks halve that on twice the workgroups, and the pair of workgroups that shares a
  // tile (linear indices 8 x groups apart) runs on one XCD, so the second reads its weights from L2.
  // Each row's arithmetic is unchanged (same k partition and sums): the same bits.
  const bool half = a.M > 16 && a.M <= 32 && ((pol.os_half >> cfg) & 1) && o.nt == 1;
  const int mt = a.M <= 16 || half ? 1 : 2;
  p.mrows = 32;
  if (o.nt > 0 && a.M <= 32 && a.ntiles % o.nt == 0) {
    // the largest k split <= the preferred one that divides the k steps, raised until every wave's share
    // fits the kernel's KPW steps; the activation slice must fit the staging (kps * MT * 64 fragments
    // <= 512 threads x 12)
    int split = 0;
    for (int d = std::min(o.split, a.KS); d >= 1; --d)
      if (a.KS % d == 0) { split = d; break; }
    while (split > 0 && split <= a.KS && (a.KS % split != 0 || a.KS / split > 8 * o.kpw)) ++split;
    if (split > 0 && split <= a.KS && (a.KS / split) * mt <= 96) {
      p.kind = GK_ONESHOT;
      p.ksplit = split;
      if (half && split == 1) {
        p.mrows = 16;
        p.mchunks = 2;
      }
    }
  }
  if (p.kind != GK_ONESHOT) p.ksplit = stream_split;
  a.kps = a.KS / p.ksplit;
  const int tiles = p.kind == GK_ONESHOT ? o.nt : streaming_tiles(cfg);
  p.tiles_per_wg = tiles;
  p.groups = (a.ntiles + tiles - 1) / tiles;
  p.part_floats = p.ksplit > 1 ? (size_t)p.groups * p.mchunks * p.ksplit * tiles * 2 * 64 * 4 : 0;
  a.ngroups = p.groups;
  // The lm_head's 256-column groups stream 768 KB of weights each (1.5B: 594 groups).  On 256 compute units
  // whole rounds give every unit two and the last 82 units a third, which sets the launch time; split over
  // three workgroups in k, those 82 groups add a third of a group to 246 units instead (measured at 32 rows:
  // 512 groups alone 76 us, all 594 98 us).  The splits meet in the last arriver, which adds them in split
  // order and runs the epilogue.
  a.tail_full = a.tail_split = 0;
  if (cfg == CFG_LM_HEAD && p.kind == GK_STREAM && p.ksplit == 1 && p.mchunks == 1 && pol.lm_tail_cus > 0) {
    const int full = p.groups / pol.lm_tail_cus * pol.lm_tail_cus, rem = p.groups - full;
    int s = rem > 0 ? std::min(3, pol.lm_tail_cus / rem) : 0;
    while (s > 1 && a.KS % s != 0) --s;
    if (s > 1) {
      a.tail_full = full;
      a.tail_split = s;
      p.part_floats = (size_t)rem * s * tiles * 2 * 64 * 4;
    }
  }
  p.tail_full = a.tail_full;
  p.tail_split = a.tail_split;
  return p;
}

template <int DT, class C, int MT>
static hipError_t launch_cfg(const GemmP& a, const GemmPlan& p, hipStream_t st) {
  size_t lds = 0;
  if (C::kw > 1) lds = (size_t)(C::kw - 1) * C::tw * C::tpw * MT * 64 * 16;
  if (C::epi == EPI_LOGITS) lds = (size_t)32 * 256 * 4;
  auto kern = gemm_pk_kernel<DT, C::epi, C::xf, MT, C::tpw, C::tw, C::kw, C::u>;
  const int gx = p.tail_split > 1 ? p.tail_full + (p.groups - p.tail_full) * p.tail_split : p.groups;
  hipLaunchKernelGGL(kern, dim3(gx, p.ksplit, p.mchunks), dim3(64 * C::tw * C::kw), lds, st, a);
  return hipGetLastError();
}

template <int DT, class C, int MT>
static hipError_t launch_os(const GemmP& a, const GemmPlan& p, hipStream_t st) {
  const size_t lds = std::max((size_t)a.kps * MT * 1024 + (size_t)a.kps * 64, (size_t)8 * C::nt * MT * 1024);
  auto kern = gemm_os_kernel<DT, C::epi, C::xf, MT, C::nt, C::kpw>;
  static size_t attr_lds = 0;  // per instantiation
  if (lds > 64 * 1024 && lds > attr_lds) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) ==
        hipSuccess)
      attr_lds = lds;
    else
      (void)hipGetLastError();
  }
  hipLaunchKernelGGL(kern, dim3(p.groups, p.ksplit, p.mchunks), dim3(512), lds, st, a);
  if (p.ksplit > 1 && a.gw.cnt == nullptr) {
    constexpr int units = (C::epi == EPI_SILU_PAIR ? C::nt / 2 : C::nt) * MT;
    hipLaunchKernelGGL((gemm_os_epilogue_kernel<DT, C::epi, MT, C::nt>), dim3(p.groups, 1, p.mchunks), dim3(64 * units), 0,
                       st, a, p.ksplit);
  }
  return hipGetLastError();
}

template <int DT, int EPI, class W>
static hipError_t launch_wr_cfg(const GemmP& a, const GemmPlan& p, hipStream_t st) {
  constexpr size_t lds = EPI == EPI_LOGITS ? std::max(W::lds, W::lds_logits) : W::lds;
  static_assert(lds <= 64 * 1024, "no LDS attribute needed");
  auto kern = gemm_wr_kernel<DT, EPI, W::mf, W::tpw, W::d>;
  const int total = p.nbm * p.nbn, per = (total + 7) / 8;
  hipLaunchKernelGGL(kern, dim3(8 * per, p.ksplit), dim3(256), lds, st, a, p.nbm, p.nbn);
  if (p.ksplit > 1 && !a.part_rows) {
    const int nblk = (a.M + 15) / 16;
    hipLaunchKernelGGL((gemm_mm_split_epilogue_kernel<DT, EPI>), dim3((a.N + 15) / 16, (nblk + 3) / 4), dim3(256), 0,
                       st, a, p.ksplit);
  }
  return hipGetLastError();
}

template <int DT, int EPI, int XF, class M>
static hipError_t launch_mm_cfg(const GemmP& a, const GemmPlan& p, hipStream_t st) {
  auto kern = gemm_mm_kernel<DT, EPI, XF, M::mf, M::tpw, M::nwm, M::nwn, M::kss, M::wd>;
  const int total = p.nbm * p.nbn, per = (total + 7) / 8;
  const size_t lds = EPI == EPI_LOGITS ? std::max(M::lds, M::lds_logits) : M::lds;
  hipLaunchKernelGGL(kern, dim3(8 * per, p.ksplit), dim3(64 * M::nw), lds, st, a, p.nbm, p.nbn);
  if (p.ksplit > 1 && !a.part_rows) {
    const int nblk = (a.M + 15) / 16;
    hipLaunchKernelGGL((gemm_mm_split_epilogue_kernel<DT, EPI>), dim3((a.N + 15) / 16, (nblk + 3) / 4), dim3(256), 0,
                       st, a, p.ksplit);
  }
  return hipGetLastError();
}

template <int DT, int EPI, class W>
static hipError_t launch_wt_cfg(const GemmP& a, const GemmPlan& p, hipStream_t st) {
  auto kern = gemm_wt_kernel<DT, EPI, W::mf, W::tpw, W::wm, W::wn, W::nbuf>;
  static bool attr = false;  // per instantiation
  if (!attr) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)W::lds) !=
        hipSuccess)
      (void)hipGetLastError();
    attr = true;
  }
  const int total = p.nbm * p.nbn, per = (total + 7) / 8;
  hipLaunchKernelGGL(kern, dim3(8 * per, p.ksplit), dim3(64 * W::nw), W::lds, st, a, p.nbm, p.nbn);
  if (p.ksplit > 1 && !a.part_rows) {
    const int nblk = (a.M + 15) / 16;
    hipLaunchKernelGGL((gemm_mm_split_epilogue_kernel<DT, EPI>), dim3((a.N + 15) / 16, (nblk + 3) / 4), dim3(256), 0,
                       st, a, p.ksplit);
  }
  return hipGetLastError();
}

// GK_MM rows arrive normalised (see GemmKind), so every large-M launch runs without the norm transform.
template <int DT, int CFG, class C>
static hipError_t launch_mm(const GemmP& a, const GemmPlan& p, hipStream_t st) {
  if (p.mm_id == MM_WR) return launch_wr_cfg<DT, C::epi, WrBig>(a, p, st);
  if (p.mm_id == MM_WR_S) {
    if constexpr (CFG != CFG_LM_HEAD) return launch_wr_cfg<DT, C::epi, WrSmall>(a, p, st);
    return hipErrorInvalidValue;
  }
  if (p.mm_id == MM_WR_T) {
    if constexpr (CFG == CFG_QKV || CFG == CFG_OPROJ) return launch_wr_cfg<DT, C::epi, WrTiny>(a, p, st);
    return hipErrorInvalidValue;
  }
  if (p.mm_id == MM_WR_M) {
    if constexpr (CFG == CFG_GATE_UP || CFG == CFG_DOWN) return launch_wr_cfg<DT, C::epi, WrMid>(a, p, st);
    return hipErrorInvalidValue;
  }
  if (p.mm_id == MM_WR_3) {
    if constexpr (CFG == CFG_OPROJ || CFG == CFG_DOWN) return launch_wr_cfg<DT, C::epi, WrB3>(a, p, st);
    return hipErrorInvalidValue;
  }
  if constexpr (CFG == CFG_GATE_UP) {
    if (p.mm_id == MM_WT_256) return launch_wt_cfg<DT, C::epi, WtB256>(a, p, st);
    if (p.mm_id == MM_WT) return launch_wt_cfg<DT, C::epi, WtBig>(a, p, st);
    if (p.mm_id == MM_WT_8) return launch_wt_cfg<DT, C::epi, WtBig8>(a, p, st);
    if (p.mm_id == MM_BIG) return launch_mm_cfg<DT, C::epi, XF_NONE, MmBig>(a, p, st);
    return launch_mm_cfg<DT, C::epi, XF_NONE, MmWide>(a, p, st);
  } else if constexpr (CFG == CFG_DOWN) {
    if (p.mm_id == MM_WT) return launch_wt_cfg<DT, C::epi, WtBig>(a, p, st);
    if (p.mm_id == MM_WT_8) return launch_wt_cfg<DT, C::epi, WtBig8>(a, p, st);
    if (p.mm_id == MM_WIDE_D) return launch_mm_cfg<DT, C::epi, XF_NONE, MmWideD>(a, p, st);
    return launch_mm_cfg<DT, C::epi, XF_NONE, MmSmall>(a, p, st);
  } else if constexpr (CFG == CFG_QKV || CFG == CFG_OPROJ) {
    return launch_mm_cfg<DT, C::epi, XF_NONE, MmSmall>(a, p, st);
  } else {
    return launch_mm_cfg<DT, C::epi, XF_NONE, MmWide>(a, p, st);  // the lm_head
  }
}

template <int DT, int CFG, class C, class O>
static hipError_t launch_mt(const GemmP& a, const GemmPlan& p, hipStream_t st) {
  if (p.kind == GK_MM) return launch_mm<DT, CFG, C>(a, p, st);
  if constexpr (O::nt > 0) {
    if (p.kind == GK_ONESHOT) {
      if (a.M <= 16 || p.mrows == 16) return launch_os<DT, O, 1>(a, p, st);
      return launch_os<DT, O, 2>(a, p, st);
    }
  }
  if (a.M <= 16) return launch_cfg<DT, C, 1>(a, p, st);
  return launch_cfg<DT, C, 2>(a, p, st);
}

template <int DT>
static hipError_t launch_dt(int cfg, const GemmP& a, const GemmPlan& p, hipStream_t st) {
  switch (cfg) {
    case CFG_QKV: return launch_mt<DT, CFG_QKV, CfgQkv, OsQkv>(a, p, st);
    case CFG_OPROJ: return launch_mt<DT, CFG_OPROJ, CfgOproj, OsOproj>(a, p, st);
    case CFG_GATE_UP: return launch_mt<DT, CFG_GATE_UP, CfgGateUp, OsGateUp>(a, p, st);
    case CFG_DOWN: return launch_mt<DT, CFG_DOWN, CfgDown, OsDown>(a, p, st);
    case CFG_LM_HEAD: return launch_mt<DT, CFG_LM_HEAD, CfgLmHead, OsNone>(a, p, st);
    default: return hipErrorInvalidValue;
  }
}

// gemm_os_kernel's dispatch: up to 4 tiles per workgroup, or gate_up without a k split, take the
// register-fragment body
bool gemm_takes_frag(int cfg, const GemmPlan& p) {
  const int nt = os_info(cfg).nt;
  return p.kind == GK_ONESHOT && p.mchunks * p.mrows <= 32 && nt > 0 && (nt <= 4 || (cfg == CFG_GATE_UP && p.ksplit == 1));
}

bool gemm_takes_blocks(const GemmPlan& p) {
  return p.kind == GK_MM && p.mm_id >= MM_WT;
}

// (the 64-row blocks only: on the 128 x 256 blocks, which have no registers left to request the table
// early, the 8192-row prefill took 30.30 against 30.16 ms with the separate pass)
bool gemm_ropes_in_epilogue(int cfg, const GemmPlan& p) {
  return cfg == CFG_QKV && p.kind == GK_MM && p.ksplit == 1 && (p.mm_id == MM_WR_T || p.mm_id == MM_WR_S);
}

hipError_t launch_gemm(int dt, int cfg, const GemmP& a, const GemmPlan& p, hipStream_t st) {
  if (a.part_rows && (p.kind != GK_MM || a.N % 4)) return hipErrorInvalidValue;
  if ((a.xfrag == 1 || a.yfrag == 1) && !gemm_takes_frag(cfg, p)) return hipErrorInvalidValue;
  if ((a.xfrag == 2 || a.yfrag == 2) && !gemm_takes_blocks(p)) return hipErrorInvalidValue;
  if (a.yfrag == 2 && cfg != CFG_GATE_UP) return hipErrorInvalidValue;
  if (a.ro.rope != nullptr && !(gemm_ropes_in_epilogue(cfg, p) && a.ntiles % 8 == 0 && a.ro.rows > 0)) return hipErrorInvalidValue;
  // a k split summed inside the launch: only the register-fragment body does it
  if (a.gw.cnt != nullptr && !(gemm_takes_frag(cfg, p) && p.ksplit > 1 && os_info(cfg).nt <= 4 && cfg != CFG_GATE_UP))
    return hipErrorInvalidValue;
  if (dt == DT_BF16) return launch_dt<DT_BF16>(cfg, a, p, st);
  return launch_dt<DT_F16>(cfg, a, p, st);
}

hipError_t launch_pack(const uint16_t* src, int N, int K, int ntiles, int mode, uint16_t* dst, hipStream_t st) {
  const size_t total = (size_t)ntiles * (K / 32) * 64;
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, src, N, K, total, mode, dst);
  return hipGetLastError();
}

hipError_t launch_confidence_combine(const float* sm, const int32_t* sa, const float* ss, int tiles, int rows,
                                     int32_t* ids, float* maxp, hipStream_t st) {
  hipLaunchKernelGGL(confidence_combine_kernel, dim3(rows), dim3(64), 0, st, sm, sa, ss, tiles, rows, ids, maxp);
  return hipGetLastError();
}

hipError_t launch_confidence_tiles(const float* logits, int ld, int vocab, int rows, float* sm, int32_t* sa,
                                   float* ss, hipStream_t st) {
  const int tiles = (vocab + 255) / 256;
  hipLaunchKernelGGL(confidence_tiles_kernel, dim3(tiles, rows), dim3(64), 0, st, logits, ld, vocab, tiles, sm, sa, ss);
  return hipGetLastError();
}

}  // namespace fdllm
