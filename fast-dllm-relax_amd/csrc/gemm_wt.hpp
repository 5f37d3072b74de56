// Large-M GEMM with both operands staged through LDS by the gfx950 global-to-LDS copy (prefill, stateless
// forward, batched steps): Y[M, N] = X[M, K] . W[N, K]^T on MFMA 16x16x32, fp32 accumulation, the
// skinny kernels' epilogues and rounding points.
//
// A workgroup of WM x WN waves computes BM = 16 MF WM rows by BNT = TPW WN weight tiles (16 columns
// each).  Wave (wm, wn) owns an MF x TPW block of 16 x 16 accumulators (128 x 96 at MF 8, TPW 6, kept
// in the accumulation registers), so each 1 KB operand fragment it reads from LDS feeds TPW or MF
// MFMAs.  The k loop runs one k step (32 columns) per stage.  A stage is BMB = MF WM activation
// fragment blocks and BNT packed weight blocks, 1 KB each, copied global -> LDS without passing through
// registers (one block per wave instruction: lane l's 16 bytes land at byte 16 l, which is MFMA
// fragment order for both: the packed weights already are, and lane l of an activation block reads row
// l % 16, columns 8 (l / 16) .. + 7).  NBUF stage buffers rotate: a wave waits for its own copies of the
// next stage (memory counter), one barrier makes every wave's copies visible and frees the buffer whose
// fragments every wave has read into registers, which then receives the copies NBUF stages ahead; the
// fragment reads of stage st + 1 overlap the MFMAs of stage st.  Every copy is unconditional
// (stages past the last re-read the last; rows past M re-read row M - 1), so every wave issues the same
// number per stage and the counter waits are exact.  When the waves do not divide a stage's blocks, the
// first SB % NW waves copy one block more than the rest, and each wave waits for its own count.
//
// K splits (gridDim.y > 1) store fp32 sums per (tile, 16-row block) exactly as gemm_mm_kernel does, and
// gemm_mm_split_epilogue_kernel adds them in split order.  Per output element the k steps are
// accumulated in order by one MFMA chain, as in the other kernels, so for the same split the results are
// the same bits as gemm_mm_kernel's.  Rows arrive normalised (the large-M path runs norm_rows once).
#pragma once
#include "gemm_mm.hpp"

namespace fdllm {

template <int DT, int EPI, int MF, int TPW, int WM, int WN, int NBUF>
__global__ __launch_bounds__(64 * WM * WN) void gemm_wt_kernel(GemmP a, int nbm, int nbn) {
  constexpr int NW = WM * WN;
  constexpr int BMB = MF * WM;        // activation blocks (16 rows) per stage
  constexpr int BNT = TPW * WN;       // weight tiles per stage
  constexpr int SB = BMB + BNT;       // 1 KB blocks per stage
  constexpr int DPW = (SB + NW - 1) / NW;  // copies per wave per stage (waves >= NHI: one fewer)
  constexpr int NHI = SB % NW == 0 ? NW : SB % NW;
  static_assert(NBUF >= 2, "at least two stage buffers");
  static_assert((NBUF - 1) * DPW < 64, "outstanding copies fit the memory counter");
  static_assert(EPI != EPI_SILU_PAIR || TPW % 2 == 0, "gate/up pairs stay within a wave");
  static_assert(EPI != EPI_LOGITS, "the lm_head takes the streaming kernel");
  extern __shared__ __align__(16) unsigned char smem[];  // [NBUF][SB][1 KB]

  const int total = nbm * nbn;
  const int per = (total + 7) / 8;
  // workgroups of one weight column block on one XCD (the hardware deals workgroups to the 8 XCDs
  // round-robin), so the blocks that re-read those weights share its L2
  const int logical = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (logical >= total) return;
  const int nb = logical / nbm, mb = logical - nb * nbm;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // wave-uniform: scalar branches
  const int wm = w / WN, wn = w - wm * WN;
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = mb * 16 * BMB, mlast = a.M - 1;
  const bool lo = NHI < NW && w >= NHI;  // this wave copies DPW - 1 blocks per stage
  const int t0 = nb * BNT, tlast = a.ntiles - 1;
  const int nst = a.KS / (int)gridDim.y;        // k steps of this split
  const int kb = (int)blockIdx.y * nst;         // its first k step

  // this wave's copies: block i = w + NW q of every stage; the per-lane source of k step 0
  const u16* src[DPW];
  size_t sstep[DPW];  // elements per k step
#pragma unroll
  for (int q = 0; q < DPW; ++q) {
    const int i = min(w + NW * q, SB - 1);  // (a low wave's last slot: never copied)
    if (i < BMB && a.xfrag == 2) {
      // fragment blocks: one 1 KB read per block (a block past the last row block re-reads the last)
      const int b = min(m0 / 16 + i, mlast / 16);
      src[q] = a.X + ((size_t)b * a.KS + kb) * 512 + 8 * lane;
      sstep[q] = 512;
    } else if (i < BMB) {
      const int m = min(m0 + 16 * i + lr, mlast);
      src[q] = a.X + (size_t)m * a.ldx + 32 * kb + 8 * lg;
      sstep[q] = 32;
    } else {
      src[q] = a.W + ((size_t)min(t0 + i - BMB, tlast) * a.KS + kb) * 512 + 8 * lane;
      sstep[q] = 512;
    }
  }
  auto copy_stage = [&](int st, int buf) {
    const int s = min(st, nst - 1);
#pragma unroll
    for (int q = 0; q < DPW; ++q)
      if (q < DPW - 1 || !lo) lds_copy16(src[q] + (size_t)s * sstep[q], smem + ((size_t)buf * SB + w + NW * q) * 1024);
  };
  // this wave's own copies of the next N stages have landed (its count per stage is DPW or DPW - 1)
  auto wait_stages = [&](auto nc) __attribute__((always_inline)) {
    constexpr int N = decltype(nc)::value;
    if (lo) wait_vmcnt<N * (DPW - 1)>();
    else wait_vmcnt<N * DPW>();
  };

  f32x4 acc[TPW][MF];
#pragma unroll
  for (int j = 0; j < TPW; ++j)
#pragma unroll
    for (int f = 0; f < MF; ++f) acc[j][f] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Stage s lives in buffer s % NBUF.  A wave reads the fragments of stage st + 1 from LDS into one
  // register set while its MFMAs consume stage st from the other, so the LDS latency hides behind the
  // MFMAs; it waits for those reads before the next barrier, after which the buffer of stage st (read one
  // iteration earlier by every wave) takes the copies of stage st + NBUF.
#pragma unroll
  for (int st = 0; st < NBUF; ++st) copy_stage(st, st);
  const u32x4* lds = reinterpret_cast<const u32x4*>(smem);
  auto read_frags = [&](u32x4 (&fr)[MF + TPW], int s) __attribute__((always_inline)) {
    const u32x4* blk = lds + (size_t)(s % NBUF) * SB * 64;
#pragma unroll
    for (int f = 0; f < MF; ++f) fr[f] = blk[(wm * MF + f) * 64 + lane];
#pragma unroll
    for (int j = 0; j < TPW; ++j) fr[MF + j] = blk[(BMB + wn * TPW + j) * 64 + lane];
  };
  // iteration st: fragments of st in cur; next receives those of st + 1 (past the last stage the buffer
  // holds a re-read of the last, read and not used)
  auto step = [&](int st, u32x4 (&cur)[MF + TPW], u32x4 (&next)[MF + TPW]) __attribute__((always_inline)) {
    wait_stages(std::integral_constant<int, NBUF - 2>{});  // this wave's copies of stage st + 1 have landed
    __builtin_amdgcn_s_barrier();    // everyone's have, and every wave's reads of stage st are done
    copy_stage(st + NBUF, st % NBUF);
    read_frags(next, st + 1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int f = 0; f < MF; ++f) acc[j][f] = mfma16<DT>(cur[MF + j], cur[f], acc[j][f]);
    __builtin_amdgcn_sched_barrier(0);
    lds_wait(next);
  };
  u32x4 fa[MF + TPW], fb[MF + TPW];
  wait_stages(std::integral_constant<int, NBUF - 1>{});  // stage 0
  __builtin_amdgcn_s_barrier();
  read_frags(fa, 0);
  lds_wait(fa);
  int st = 0;
#pragma nounroll
  for (; st + 1 < nst; st += 2) {
    step(st, fa, fb);
    step(st + 1, fb, fa);
  }
  if (st < nst) step(st, fa, fb);
  wait_vmcnt<0>();  // no copy may still be writing LDS when the workgroup ends

  const int f0 = wm * MF, tw0 = t0 + wn * TPW;
  if (gridDim.y > 1) {
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int f = 0; f < MF; ++f) store_split_unit(a, blockIdx.y, tw0 + j, mb * BMB + f0 + f, lane, acc[j][f]);
    return;
  }
  if constexpr (EPI == EPI_SILU_PAIR) {
#pragma unroll
    for (int p = 0; p < TPW / 2; ++p)
#pragma unroll
      for (int f = 0; f < MF; ++f) {
        const f32x4 v[2] = {acc[2 * p][f], acc[2 * p + 1][f]};
        os_epilogue<DT, EPI, 2, false>(a, v, m0 + 16 * (f0 + f) + lr, tw0 + 2 * p, lg);
      }
  } else {
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int f = 0; f < MF; ++f) {
        const f32x4 v[1] = {acc[j][f]};
        os_epilogue<DT, EPI, 1, false>(a, v, m0 + 16 * (f0 + f) + lr, tw0 + j, lg);
      }
  }
}

// Large-M GEMM with the weights loaded straight into registers and only the activations staged in LDS.
// Same arithmetic, split partials and epilogues as gemm_wt_kernel (per output element one MFMA chain
// over the k steps in order), so for the same k split the results are the same bits.
//
// Why: in gemm_wt_kernel every operand byte crosses LDS twice (the global -> LDS copy, then one
// fragment read per wave that uses it), and LDS bandwidth (128 B per clock per compute unit) runs out
// before the MFMAs do.  Here the four waves of a workgroup share the BM = 16 MF activation rows (one
// LDS copy, four reads) and each wave owns TPW weight tiles, which no other wave needs: its packed
// 1 KB weight blocks are already in MFMA fragment order, so they go from global memory to registers
// with one coalesced 16-byte load per lane.  A block is 16 MF rows x 64 TPW columns.
//
// Pipeline: D stages in flight.  Stage st uses LDS buffer st % R and weight register set st % R
// (R = D + 1), so the copies for stage st + D, issued right after the barrier of stage st, go into the
// buffer and register set that stage st - 1 used.  In the k loop (unrolled by R so that the register sets
// are named at compile time) each stage issues exactly VPS = TPW + MF / 4 vector memory instructions per
// wave (stages past the last re-read the last), weights first, and the issue is fenced against compiler
// motion, so "all but the (D - 1) VPS most recent" is exactly "stage st has landed"; the last nst % R
// stages, after the loop, wait for all.
// The qkv epilogue with RoPE and the KV append (RopeOut): the block's sums + bias (rbias, requested early
// with the table entries rcs) rounded to the model dtype (EPI_BIAS), then per element rope_kv_kernel's arithmetic (rope_pairs: lo' = rnd(x1 c) + rnd(-x2 s), hi' =
// rnd(x2 c) + rnd(x1 s), x1 / x2 the values at dims d and d + 64 of the head, (c, s) the table entry d of
// the row) and its destinations.  The tiles arrive in perm8 order, so the partner of this wave's tile j is
// tile j of wave w ^ 1 (two tiles per wave) or w ^ 2 (one), read through the stage buffers (free once the
// k loop ended).  The same lane holds the same row and the same
// four dims of both.
template <int DT, int MF, int TPW>
__device__ __forceinline__ void wr_qkv_rope(const GemmP& a, const f32x4 (&acc)[TPW][MF], int m0, int tw0, int lane,
                                            int w, unsigned char* smem, const f32x4 (&rcs)[TPW][MF][2],
                                            const u32x2 (&rbias)[TPW]) {
  static_assert(TPW == 1 || TPW == 2, "rotation pairs in two waves of the block");
  const int lr = lane & 15, lg = lane >> 4;
  const RopeOut& ro = a.ro;
  u32x2 x[TPW][MF];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const float bv[4] = {lo_f32<DT>(rbias[j][0]), hi_f32<DT>(rbias[j][0]), lo_f32<DT>(rbias[j][1]), hi_f32<DT>(rbias[j][1])};
#pragma unroll
    for (int f = 0; f < MF; ++f) {
      u16 out[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) out[i] = from_f32<DT>(acc[j][f][i] + bv[i]);
      x[j][f] = u32x2{pack2(out[0], out[1]), pack2(out[2], out[3])};
    }
  }
  u32x2 y[TPW][MF];
  u32x2* xb = reinterpret_cast<u32x2*>(smem);  // [4 waves][TPW][MF][64 lanes]
  __syncthreads();  // every wave is done reading the stage buffers
#pragma unroll
  for (int j = 0; j < TPW; ++j)
#pragma unroll
    for (int f = 0; f < MF; ++f) xb[((w * TPW + j) * MF + f) * 64 + lane] = x[j][f];
  __syncthreads();
  const int pw = TPW == 2 ? (w ^ 1) : (w ^ 2);
#pragma unroll
  for (int j = 0; j < TPW; ++j)
#pragma unroll
    for (int f = 0; f < MF; ++f) y[j][f] = xb[((pw * TPW + j) * MF + f) * 64 + lane];
  const size_t krow = (size_t)ro.nkv * 128;
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int t = perm8(tw0 + j);
    const int hd = t >> 3, dh = 16 * (t & 7) + 4 * lg;  // head; first of the lane's four dims in it
    const bool lo = dh < 64;
    const int dl = dh & 63;
#pragma unroll
    for (int f = 0; f < MF; ++f) {
      const int m = m0 + 16 * f + lr;
      if (m >= a.M || 16 * t >= a.N) continue;
      const int b = m / ro.rows, rl = m - b * ro.rows;
      u16* kvrow = nullptr;
      if (hd >= ro.nq) kvrow = (hd < ro.nq + ro.nkv ? ro.kc : ro.vc) + b * ro.seq_stride + (size_t)(ro.ws[b] + rl) * krow;
      if (hd >= ro.nq + ro.nkv) {
        *reinterpret_cast<u32x2*>(kvrow + (hd - ro.nq - ro.nkv) * 128 + dh) = x[j][f];
        continue;
      }
      const f32x4 t0 = rcs[j][f][0], t1 = rcs[j][f][1];
      const float cs[8] = {t0[0], t0[1], t0[2], t0[3], t1[0], t1[1], t1[2], t1[3]};
      const u32x2 v1 = lo ? x[j][f] : y[j][f], v2 = lo ? y[j][f] : x[j][f];  // dims dl .., dl + 64 ..
      const float x1[4] = {lo_f32<DT>(v1[0]), hi_f32<DT>(v1[0]), lo_f32<DT>(v1[1]), hi_f32<DT>(v1[1])};
      const float x2[4] = {lo_f32<DT>(v2[0]), hi_f32<DT>(v2[0]), lo_f32<DT>(v2[1]), hi_f32<DT>(v2[1])};
      u16 o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float c = cs[2 * i], sn = cs[2 * i + 1];
        o[i] = lo ? from_f32<DT>(rnd<DT>(x1[i] * c) + rnd<DT>(-x2[i] * sn))
                  : from_f32<DT>(rnd<DT>(x2[i] * c) + rnd<DT>(x1[i] * sn));
      }
      u16* dst = hd < ro.nq ? ro.q + (size_t)m * ro.nq * 128 + hd * 128 + dh : kvrow + (hd - ro.nq) * 128 + dh;
      *reinterpret_cast<u32x2*>(dst) = u32x2{pack2(o[0], o[1]), pack2(o[2], o[3])};
    }
  }
}

template <int DT, int EPI, int MF, int TPW, int D>
// (up to 32 accumulator tiles per wave, two workgroups per compute unit: at most 256 registers per lane,
// accumulators included; more tiles, one workgroup)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MF * TPW <= 32 ? 2 : 1, MF * TPW <= 32 ? 2 : 1)))
void gemm_wr_kernel(GemmP a, int nbm, int nbn) {
  constexpr int NW = 4, R = D + 1;
  constexpr int DPW = MF / NW;        // activation blocks each wave copies per stage
  constexpr int VPS = TPW + DPW;      // vector memory instructions per wave per stage
  static_assert(MF % NW == 0, "every wave copies the same number of activation blocks");
  static_assert(D >= 1 && (D - 1) * VPS < 64, "outstanding copies fit the memory counter");
  static_assert(EPI != EPI_SILU_PAIR || TPW % 2 == 0, "gate/up pairs stay within a wave");
  static_assert(EPI != EPI_LOGITS || NW * TPW == 16, "one 256-column confidence tile per block column");
  extern __shared__ __align__(16) unsigned char smem[];  // [R][MF][1 KB]; EPI_LOGITS: then [16 MF][256] u16

  const int total = nbm * nbn;
  const int per = (total + 7) / 8;
  // the row blocks of one weight column block on one XCD (workgroup i runs on XCD i % 8), so its
  // weights come from HBM once per XCD
  const int logical = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (logical >= total) return;
  const int nb = logical / nbm, mb = logical - nb * nbm;

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = mb * 16 * MF, mlast = a.M - 1;
  const int tw0 = (nb * NW + w) * TPW, tlast = a.ntiles - 1;  // this wave's first tile
  const int nst = a.KS / (int)gridDim.y;
  const int kb = (int)blockIdx.y * nst;

  const u16* xs[DPW];
  size_t xstep[DPW];
#pragma unroll
  for (int q = 0; q < DPW; ++q) {
    const int i = w + NW * q;
    if (a.xfrag == 2) {
      const int b = min(m0 / 16 + i, mlast / 16);
      xs[q] = a.X + ((size_t)b * a.KS + kb) * 512 + 8 * lane;
      xstep[q] = 512;
    } else {
      const int m = min(m0 + 16 * i + lr, mlast);
      xs[q] = a.X + (size_t)m * a.ldx + 32 * kb + 8 * lg;
      xstep[q] = 32;
    }
  }
  // qkv with RoPE in the epilogue takes its tiles in perm8 order (RopeOut)
  const bool rope = EPI == EPI_BIAS && a.ro.rope != nullptr;
  const u16* ws[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j)
    ws[j] = a.W + ((size_t)min(rope ? perm8(tw0 + j) : tw0 + j, tlast) * a.KS + kb) * 512 + 8 * lane;

  u32x4 wv[R][TPW];
  auto issue = [&](int st, u32x4 (&dst)[TPW], int buf) {
    const int s = min(st, nst - 1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < TPW; ++j) dst[j] = *reinterpret_cast<const u32x4*>(ws[j] + (size_t)s * 512);
#pragma unroll
    for (int q = 0; q < DPW; ++q)
      lds_copy16(xs[q] + (size_t)s * xstep[q], smem + ((size_t)buf * MF + w + NW * q) * 1024);
    __builtin_amdgcn_sched_barrier(0);
  };

  f32x4 acc[TPW][MF];
#pragma unroll
  for (int j = 0; j < TPW; ++j)
#pragma unroll
    for (int f = 0; f < MF; ++f) acc[j][f] = f32x4{0.f, 0.f, 0.f, 0.f};

  // qkv with RoPE in the epilogue: the table entries and the bias values the epilogue takes, requested
  // before the pipeline (older than every stage's copies, so stage 0's counted wait covers them)
  constexpr bool RPRE = EPI == EPI_BIAS && TPW <= 2;
  f32x4 rcs[RPRE ? TPW : 1][RPRE ? MF : 1][2];
  u32x2 rbias[RPRE ? TPW : 1];
  if constexpr (RPRE) {
    if (rope) {
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        const int t = perm8(tw0 + j), n = 16 * t + 4 * lg, dl = (16 * (t & 7) + 4 * lg) & 63;
        rbias[j] = *reinterpret_cast<const u32x2*>(a.bias + min(n, a.N - 4));
#pragma unroll
        for (int f = 0; f < MF; ++f) {
          const float* cs = a.ro.rope + (size_t)min(m0 + 16 * f + lr, mlast) * 128 + 2 * dl;
          rcs[j][f][0] = *reinterpret_cast<const f32x4*>(cs);
          rcs[j][f][1] = *reinterpret_cast<const f32x4*>(cs + 4);
        }
      }
    }
  }

#pragma unroll
  for (int u = 0; u < D; ++u) issue(u, wv[u], u);

  // stage st = st0 + u with u = st % R known at compile time.  EXACT: the D - 1 stages issued after stage
  // st each issued VPS instructions, so the count wait is exact.  The last nst % R stages (after the loop)
  // wait for everything instead: there the compiler drops the weight loads of stages past the last, whose
  // registers are never read, so fewer than VPS instructions per stage follow and a count wait would
  // return before stage st's copies landed.
  const u32x4* lds = reinterpret_cast<const u32x4*>(smem);
  // PIPE (blocks with registers to spare): a wave reads stage st + 1's activation fragments right after
  // its MFMAs of stage st are issued, so the LDS latency passes during the next wait and barrier; the
  // wait of stage st is then for stage st + 1's copies (one stage less of lead, of D).  Otherwise the
  // fragments of stage st are read after its barrier.
  constexpr bool PIPE = MF * TPW <= 16 && D >= 3;
  u32x4 xf[MF];
  if constexpr (PIPE) {
    wait_vmcnt<(D - 1) * VPS>();  // stage 0
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int f = 0; f < MF; ++f) xf[f] = lds[f * 64 + lane];
  }
  auto stage = [&](int st, auto uc, auto exact) {
    constexpr int u = decltype(uc)::value;
    if constexpr (PIPE) {
      if constexpr (decltype(exact)::value) wait_vmcnt<(D - 2) * VPS>();  // stage st + 1's copies and weights
      else wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();  // every wave's have; every wave read buffer (u - 1) % R one stage ago
    } else {
      if constexpr (decltype(exact)::value) wait_vmcnt<(D - 1) * VPS>();  // stage st's copies and weights
      else wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();    // every wave's copies have; buffer (u - 1) % R is free
    }
    issue(st + D, wv[(u + D) % R], (u + D) % R);
    if constexpr (!PIPE) {
      const u32x4* blk = lds + (size_t)u * MF * 64;
#pragma unroll
      for (int f = 0; f < MF; ++f) xf[f] = blk[f * 64 + lane];
    }
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int f = 0; f < MF; ++f) acc[j][f] = mfma16<DT>(wv[u][j], xf[f], acc[j][f]);
    if constexpr (PIPE) {
      // stage st + 1 (past the last: the copies re-read the last stage, read and not used)
      const u32x4* nblk = lds + (size_t)((u + 1) % R) * MF * 64;
#pragma unroll
      for (int f = 0; f < MF; ++f) xf[f] = nblk[f * 64 + lane];
    }
  };
  // whole rounds of R stages, then the last nst % R stages outside the loop (an exit from inside the
  // unrolled round would make the compiler's own counter bookkeeping wait for everything at its top)
  int st0 = 0;
#pragma nounroll
  for (; st0 + R <= nst; st0 += R)
    static_for<0, R>([&](auto uc) { stage(st0 + decltype(uc)::value, uc, std::true_type{}); });
  static_for<0, R - 1>([&](auto uc) {
    if (st0 + decltype(uc)::value < nst) stage(st0 + decltype(uc)::value, uc, std::false_type{});
  });
  wait_vmcnt<0>();  // no copy may still be writing LDS when the workgroup ends

  if (gridDim.y > 1) {
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int f = 0; f < MF; ++f) store_split_unit(a, blockIdx.y, tw0 + j, mb * MF + f, lane, acc[j][f]);
    return;
  }
  if constexpr (EPI == EPI_LOGITS) {
    // the lm_head: the block's logits rounded to the model dtype (cuda.py:708-711) into an LDS tile
    // (and the optional fp32 output), then the confidence statistics of its 256 columns, exactly as
    // gemm_mm_kernel does
    __syncthreads();  // every wave is done with the stage buffers the tile overwrites
    u16* tile = reinterpret_cast<u16*>(smem);
    const int n0 = nb * 256;
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int f = 0; f < MF; ++f) {
        const int ml = 16 * f + lr, nl = 16 * (w * TPW + j) + 4 * lg, n = n0 + nl, m = m0 + ml;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = rnd<DT>(acc[j][f][i]);
        *reinterpret_cast<u32x2*>(tile + ml * 256 + nl) = u32x2{pack_f32x2<DT>(v[0], v[1]), pack_f32x2<DT>(v[2], v[3])};
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
    logits_tile_stats<DT, 16 * MF, NW>(a, tile, m0, nb, w, lane);
  } else if constexpr (EPI == EPI_SILU_PAIR) {
#pragma unroll
    for (int p = 0; p < TPW / 2; ++p)
#pragma unroll
      for (int f = 0; f < MF; ++f) {
        const f32x4 v[2] = {acc[2 * p][f], acc[2 * p + 1][f]};
        os_epilogue<DT, EPI, 2, false>(a, v, m0 + 16 * f + lr, tw0 + 2 * p, lg);
      }
  } else {
    if constexpr (EPI == EPI_BIAS) {
      if constexpr (RPRE) {
        if (rope) {
          wr_qkv_rope<DT, MF, TPW>(a, acc, m0, tw0, lane, w, smem, rcs, rbias);
          return;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int f = 0; f < MF; ++f) {
        const f32x4 v[1] = {acc[j][f]};
        os_epilogue<DT, EPI, 1, false>(a, v, m0 + 16 * f + lr, tw0 + j, lg);
      }
  }
}

}  // namespace fdllm
