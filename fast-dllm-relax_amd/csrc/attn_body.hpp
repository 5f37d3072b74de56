// GQA attention of a block of rows against the in-place KV cache, with RoPE and the KV append fused in
// (fast_dllm.attn_inplace, fast_dllm_relax/runtime.py:51-73; RoPE cuda.py:278-316; in-graph restatement
// model/metal.py:255-302, 378-408).  Query head h uses kv head h / (nq / nkv); scores q.k * scale in
// fp32, online softmax in fp32 (in base 2: scores scaled by scale x log2(e), exponentials by the
// hardware exp2), P rounded to the model dtype for P.V on MFMA with fp32 accumulation (the
// flash-attention precision the reference's callback uses), one rounding of the output.  Split partials
// carry their running maxima in the same base-2 units.
//
// Rows [ws, ws + rows) of the cache belong to this call: their K (after RoPE) and V are taken straight
// from this call's qkv projection, and workgroup column 0 writes them to the cache.  Every other key
// row comes from the cache.  Queries are RoPE'd in registers at positions pos_offset + r.
//
// Work split: blockIdx.y = kv head g, blockIdx.z = key split c, blockIdx.x = group of QPW query tiles
// (the query rows of the grp heads sharing g are stacked: row qi = head_in_group * rows + r, 16 per
// tile).  The workgroup's QPW x KSW waves are QPW query-tile slots times KSW key groups; key group kg
// stages blocks of 32 keys (K row-major, V transposed four keys at a time) in its own LDS buffers and
// its waves run the scores S^T = K . Q^T and O^T += V^T . P^T for their query tiles (a lane holds one
// query, so its softmax statistics stay in-lane).  Key groups are merged in LDS in fixed order; key
// splits (S > 1) leave partials that attn_merge_kernel combines in split order, so results are
// deterministic.
#pragma once
#include "common.hpp"
#include "kernels.hpp"

namespace fdllm {

constexpr int HD = 128;
constexpr int KB = 32;        // keys per block
constexpr int KLD = HD + 8;   // u16 stride of a K row in LDS
constexpr int VLD = KB + 8;   // u16 stride of a transposed V row (one head dimension)
constexpr int PSZ = 16 * HD + 32;  // floats per split partial of one query tile: O, then (m, l) per query
constexpr float LOG2E = 1.4426950408889634f;

template <int DT> __device__ __forceinline__ float elem(const u32x4& v, int e) {
  return (e & 1) ? hi_f32<DT>(v[e >> 1]) : lo_f32<DT>(v[e >> 1]);
}

// RoPE of 8 rotation pairs: lo holds dims i0 .. i0 + 7 (< 64), hi the partner dims + 64; cs points at
// the (cos, sin) entries i0 .. i0 + 7 of the position's table row (cuda.py:314-315 with _rotate_half
// 207-209: q' = q cos + rot(q) sin, every product and sum rounded to the model dtype).
template <int DT>
__device__ __forceinline__ void rope_pairs(u32x4& lo, u32x4& hi, const f32x4 (&t)[4]) {
  u16 o1[8], o2[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float c = t[e >> 1][2 * (e & 1)], sn = t[e >> 1][2 * (e & 1) + 1];
    const float x1 = elem<DT>(lo, e), x2 = elem<DT>(hi, e);
    o1[e] = from_f32<DT>(rnd<DT>(x1 * c) + rnd<DT>(-x2 * sn));
    o2[e] = from_f32<DT>(rnd<DT>(x2 * c) + rnd<DT>(x1 * sn));
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    lo[c] = pack2(o1[2 * c], o1[2 * c + 1]);
    hi[c] = pack2(o2[2 * c], o2[2 * c + 1]);
  }
}
template <int DT>
__device__ __forceinline__ void rope_tab(u32x4& lo, u32x4& hi, const float* cs) {
  f32x4 t[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) t[c] = *reinterpret_cast<const f32x4*>(cs + 4 * c);
  rope_pairs<DT>(lo, hi, t);
}

// Output element (row r, column c = head x 128 + dim): row-major [rows][nq x 128], or MFMA-fragment
// order (frag_off) when the next projection is a one-shot chain's (at most 32 rows, one sequence).
__device__ __forceinline__ u16* out_at(const AttnP& a, int r, int c) {
  return a.out + (a.ofrag ? frag_off(r, c) : (size_t)r * a.nq * HD + c);
}

template <int DT, int QPW, int KSW>
__global__ __launch_bounds__(64 * QPW * KSW) void attn_kernel(AttnP a) {
  constexpr int NT = 64 * QPW;  // threads of one key group
  constexpr int KBUF = KB * KLD, VBUF = HD * VLD;
  extern __shared__ __align__(16) unsigned char smem[];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int qw = w % QPW, kg = w / QPW;
  const int tid = threadIdx.x - kg * NT;
  const int lr = lane & 15, lg = lane >> 4;
  const int g = blockIdx.y, c = blockIdx.z;
  const int grp = a.nq / a.nkv, QR = grp * a.rows, QT = (QR + 15) / 16;
  const int qt = blockIdx.x * QPW + qw;
  const bool tile_ok = qt < QT;
  const size_t krow = (size_t)a.nkv * HD;
  u16* kbuf = reinterpret_cast<u16*>(smem) + kg * KBUF;
  u16* vbuf = reinterpret_cast<u16*>(smem) + KSW * KBUF + kg * VBUF;

  // this lane's query row: qi = 16 qt + lr
  const int qi = qt * 16 + lr;
  const bool qvalid = tile_ok && qi < QR;
  const int hh = qvalid ? qi / a.rows : 0;
  const int r = qvalid ? qi - hh * a.rows : 0;
  u32x4 qf[4];
  {
    const u16* qp = a.qkv + (size_t)r * a.ldq + (g * grp + hh) * HD + 8 * lg;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
      qf[ds] = qvalid ? *reinterpret_cast<const u32x4*>(qp + 32 * ds) : u32x4{0u, 0u, 0u, 0u};
    if (a.rope != nullptr) {  // null: the queries arrive rotated (fdllm_attn_inplace)
      const float* cs = a.rope + (size_t)r * 128;
      rope_tab<DT>(qf[0], qf[2], cs + 16 * lg);
      rope_tab<DT>(qf[1], qf[3], cs + 16 * lg + 64);
    }
  }
  const int qpos_blk = a.mask == 1 ? (a.q_pos0 + r) / a.block : 0;
  const float* brow = a.mask == 2 ? a.bias + (long long)r * a.bias_ld : nullptr;
  const float c2 = a.scale * LOG2E;

  const int kbeg = c * a.chunk;
  const int kend = min(kbeg + a.chunk, a.Lk);
  const int nblk = (kend - kbeg + KB - 1) / KB;
  const int iters = (nblk + KSW - 1) / KSW;
  const bool writer = blockIdx.x == 0;
  const u16* kq_base = a.qkv + a.nq * HD + g * HD;
  const u16* vq_base = a.qkv + (a.nq + a.nkv) * HD + g * HD;

  float m_run = -INFINITY, l_run = 0.f;
  f32x4 o[HD / 16];
#pragma unroll
  for (int dt = 0; dt < HD / 16; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int it = 0; it < iters; ++it) {
    const int b = it * KSW + kg;
    const int kb = kbeg + b * KB;
    const bool bvalid = b < nblk;
    __syncthreads();
    if (bvalid) {
      // K: 32 keys x 8 rotation-pair chunks
      for (int item = tid; item < KB * 8; item += NT) {
        const int j = item >> 3, p = item & 7;
        const int key = kb + j;
        u32x4 lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
        if (key < kend) {
          if (key >= a.ws && key < a.ws + a.rows) {
            const u16* src = kq_base + (size_t)(key - a.ws) * a.ldq;
            lo = *reinterpret_cast<const u32x4*>(src + 8 * p);
            hi = *reinterpret_cast<const u32x4*>(src + 64 + 8 * p);
            rope_tab<DT>(lo, hi, a.rope + (size_t)(key - a.ws) * 128 + 16 * p);
            if (writer) {
              u16* dst = a.kc + key * krow + g * HD;
              *reinterpret_cast<u32x4*>(dst + 8 * p) = lo;
              *reinterpret_cast<u32x4*>(dst + 64 + 8 * p) = hi;
            }
          } else {
            const u16* src = a.kc + key * krow + g * HD;
            lo = *reinterpret_cast<const u32x4*>(src + 8 * p);
            hi = *reinterpret_cast<const u32x4*>(src + 64 + 8 * p);
          }
        }
        *reinterpret_cast<u32x4*>(kbuf + j * KLD + 8 * p) = lo;
        *reinterpret_cast<u32x4*>(kbuf + j * KLD + 64 + 8 * p) = hi;
      }
      // V: 8 key quads x 16 dim chunks, stored transposed (vbuf[dim][key], four keys per 8-byte word)
      for (int item = tid; item < 8 * 16; item += NT) {
        const int kq = item >> 4, dc = item & 15;
        u32x4 v[4];
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int key = kb + 4 * kq + qq;
          v[qq] = u32x4{0u, 0u, 0u, 0u};
          if (key < kend) {
            if (key >= a.ws && key < a.ws + a.rows) {
              v[qq] = *reinterpret_cast<const u32x4*>(vq_base + (size_t)(key - a.ws) * a.ldq + 8 * dc);
              if (writer) *reinterpret_cast<u32x4*>(a.vc + key * krow + g * HD + 8 * dc) = v[qq];
            } else {
              v[qq] = *reinterpret_cast<const u32x4*>(a.vc + key * krow + g * HD + 8 * dc);
            }
          }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int sh = 16 * (e & 1);
          const unsigned long long wd =
              (unsigned long long)((v[0][e >> 1] >> sh) & 0xffffu) |
              ((unsigned long long)((v[1][e >> 1] >> sh) & 0xffffu) << 16) |
              ((unsigned long long)((v[2][e >> 1] >> sh) & 0xffffu) << 32) |
              ((unsigned long long)((v[3][e >> 1] >> sh) & 0xffffu) << 48);
          *reinterpret_cast<unsigned long long*>(vbuf + (8 * dc + e) * VLD + 4 * kq) = wd;
        }
      }
    }
    __syncthreads();
    if (!bvalid || !tile_ok) continue;

    f32x4 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
      const u16* kp = kbuf + (16 * kt + lr) * KLD + 8 * lg;
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) s[kt] = mfma16<DT>(*reinterpret_cast<const u32x4*>(kp + 32 * ds), qf[ds], s[kt]);
    }
    // lane holds S^T[key = kb + 16 kt + 4 lg + i][query lr]
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kb + 16 * kt + 4 * lg + i;
        float v = s[kt][i] * c2;
        if (key >= kend) {
          v = -INFINITY;
        } else if (a.mask == 1) {
          if (qpos_blk < key / a.block) v = -INFINITY;
        } else if (a.mask == 2) {
          v += brow[key] * LOG2E;
        }
        s[kt][i] = v;
        mx = fmaxf(mx, v);
      }
    mx = rows_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float ps = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(s[kt][i] - m_use);
        s[kt][i] = p;
        ps += p;
      }
    ps = rows_sum(ps);
    l_run = l_run * alpha + ps;
    m_run = m_new;
    // P^T as the B operand: k slot 8 lg + e holds key 4 lg + e (e < 4) or 16 + 4 lg + e - 4 (e >= 4);
    // the V^T fragment (A operand) reads the same keys; O^T accumulates with this lane's query lr
    const u32x4 pa = {pack2(from_f32<DT>(s[0][0]), from_f32<DT>(s[0][1])),
                      pack2(from_f32<DT>(s[0][2]), from_f32<DT>(s[0][3])),
                      pack2(from_f32<DT>(s[1][0]), from_f32<DT>(s[1][1])),
                      pack2(from_f32<DT>(s[1][2]), from_f32<DT>(s[1][3]))};
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt) {
      const u16* vrow = vbuf + (16 * dt + lr) * VLD + 4 * lg;
      const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
      const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 16);
      o[dt] = mfma16<DT>(u32x4{lo[0], lo[1], hi[0], hi[1]}, pa, o[dt] * alpha);
    }
  }

  // ---- merge the key groups in LDS (fixed order kg = 0, 1, ...); lane holds O^T[dims][query lr] ----
  float Mq, Lq;
  __syncthreads();
  {
    float* cm = reinterpret_cast<float*>(smem);
    float* cl = cm + KSW * QPW * 16;
    f32x4* co = reinterpret_cast<f32x4*>(cl + KSW * QPW * 16);
    if (lg == 0) {
      cm[(kg * QPW + qw) * 16 + lr] = m_run;
      cl[(kg * QPW + qw) * 16 + lr] = l_run;
    }
    if (KSW > 1 && kg > 0) {
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt) co[(((kg - 1) * QPW + qw) * (HD / 16) + dt) * 64 + lane] = o[dt];
    }
    __syncthreads();
    if (kg == 0) {
      float M = -INFINITY;
      for (int k2 = 0; k2 < KSW; ++k2) M = fmaxf(M, cm[(k2 * QPW + qw) * 16 + lr]);
      const float Mu = M == -INFINITY ? 0.f : M;
      float L = 0.f;
      for (int k2 = 0; k2 < KSW; ++k2) L += cl[(k2 * QPW + qw) * 16 + lr] * __builtin_amdgcn_exp2f(cm[(k2 * QPW + qw) * 16 + lr] - Mu);
      const float f0 = __builtin_amdgcn_exp2f(cm[qw * 16 + lr] - Mu);
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt) o[dt] *= f0;
      for (int k2 = 1; k2 < KSW; ++k2) {
        const float fk = __builtin_amdgcn_exp2f(cm[(k2 * QPW + qw) * 16 + lr] - Mu);
#pragma unroll
        for (int dt = 0; dt < HD / 16; ++dt) o[dt] += co[(((k2 - 1) * QPW + qw) * (HD / 16) + dt) * 64 + lane] * fk;
      }
      Mq = M;
      Lq = L;
    }
  }
  if (kg != 0 || !tile_ok) return;
  if (a.S == 1) {
    if (qvalid) {
      const float inv = 1.0f / Lq;
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt)
        *reinterpret_cast<u32x2*>(out_at(a, r, (g * grp + hh) * HD + 16 * dt + 4 * lg)) =
            u32x2{pack2(from_f32<DT>(o[dt][0] * inv), from_f32<DT>(o[dt][1] * inv)),
                  pack2(from_f32<DT>(o[dt][2] * inv), from_f32<DT>(o[dt][3] * inv))};
    }
    return;
  }
  // key splits: the partial of (g, qt, c) in the layout attn_merge_kernel reads
  float* pp = a.part + ((size_t)(g * QT + qt) * a.S + c) * PSZ;
#pragma unroll
  for (int dt = 0; dt < HD / 16; ++dt) reinterpret_cast<f32x4*>(pp)[dt * 64 + lane] = o[dt];
  if (lg == 0) *reinterpret_cast<f32x2_t*>(pp + 16 * HD + 2 * lr) = f32x2_t{Mq, Lq};
}

// ---- one-shot variant for short key chunks (the cached decode step) -------------------------------
// Same arithmetic as attn_kernel, but a workgroup requests every K/V row of its chunk (CH keys) at
// once, so the chunk costs one memory latency instead of one per 32-key block.  Waves are QPW query
// tiles times KH key parts.  The output is accumulated transposed, O^T = V^T P^T, so that a lane holds
// one query (its softmax statistics stay in-lane) and the row reductions use row-swap permutes.  The
// key parts are merged in LDS; with key splits (more than one chunk) each workgroup stores its partial
// and attn_merge_kernel, launched next on the stream, combines them across many workgroups.  (Merging
// them inside this launch, the chunks of a (query-tile group, kv head) meeting at a group counter, was
// bit-identical but slower: 15.0 us against 10.5 + 4.0 us at 32 rows and prefix 2048, 17.5 against
// 7.6 + 4.8 us at 8 rows.)
// Body of one workgroup (query-tile group bx, kv head by, key chunk bz; tid = threadIdx.x), in two phases:
// attn_chunk_load requests the chunk's K/V rows into registers (AttnChunkRegs) and attn_chunk_compute
// does the rest.

// WCS: also hold the RoPE (cos, sin) entries of items whose key is one of this call's rows, requested
// with the K/V
template <int QPW, int KH, int CH, bool WCS = false>
struct AttnChunkRegs {
  static constexpr int NT = 64 * QPW * KH;
  static constexpr int KIT = (CH * 8 + NT - 1) / NT;        // K items (rotation-pair chunks) per thread
  static constexpr int VIT = ((CH / 4) * 16 + NT - 1) / NT;  // V items (key quad x dim chunk) per thread
  static constexpr bool wcs = WCS;
  u32x4 klo[KIT], khi[KIT], vv[VIT][4];
  f32x4 kcs[WCS ? KIT : 1][4];
  u32x4 qf[4];        // the lane's query (before RoPE) and its RoPE table entries, requested first
  f32x4 qcs[2][4];
};

// The lane's query row and its RoPE (cos, sin) entries, requested before the chunk's K/V: a wave's loads
// issue only as fast as the compute unit takes data in, and requested after the 64 KB of K/V (as they
// were) they landed last and the query RoPE waited for all of it.
template <int QPW, int KH, int CH, bool WCS>
__device__ __forceinline__ void attn_chunk_qload(const AttnP& a, int bx, int by, AttnChunkRegs<QPW, KH, CH, WCS>& R,
                                                 int tid) {
  const int lane = tid & 63, w = tid >> 6;
  const int qw = w % QPW, kh = w / QPW;
  const int lr = lane & 15, lg = lane >> 4;
  const int grp = a.nq / a.nkv, QR = grp * a.rows, QT = (QR + 15) / 16;
  const int qt = bx * QPW + qw;
  const int qi = qt * 16 + lr;
  const bool qvalid = qt < QT && qi < QR;
  const int hh = qvalid ? qi / a.rows : 0;
  const int r = qvalid ? qi - hh * a.rows : 0;
  const bool qshare = KH > 1 && a.nseq <= 1;
  if (!qshare || kh == 0) {
    const u16* qp = a.qkv + (size_t)r * a.ldq + (by * grp + hh) * HD + 8 * lg;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) R.qf[ds] = ld16<false>(qp + 32 * ds);
    if (a.rope != nullptr) {  // null: the queries arrive rotated (fdllm_attn_inplace)
      const float* cs = a.rope + (size_t)r * 128 + 16 * lg;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        R.qcs[0][c] = *reinterpret_cast<const f32x4*>(cs + 4 * c);
        R.qcs[1][c] = *reinterpret_cast<const f32x4*>(cs + 64 + 4 * c);
      }
    }
  }
}

// Item -> (key, chunk) maps: 16 consecutive lanes take 16 keys of one K chunk (with, for this call's own
// rows, the key's RoPE table entries, so the RoPE at staging waits for no further load), and 32
// consecutive lanes take 16 key quads x 2 dim chunks of V, so the LDS stores of attn_chunk_compute hit 64 distinct banks
// per pass (rows are 68 dwords apart, 4 banks on).  Rows past kend read row kbeg and are masked or
// zeroed later.
template <int QPW, int KH, int CH, bool WCS = false>
__device__ __forceinline__ void attn_chunk_load(const AttnP& a, int by, int bz, AttnChunkRegs<QPW, KH, CH, WCS>& R,
                                                int tid) {
  typedef AttnChunkRegs<QPW, KH, CH, WCS> Regs;
  constexpr int NT = Regs::NT, KIT = Regs::KIT, VIT = Regs::VIT;
  const int g = by;
  const size_t krow = (size_t)a.nkv * HD;
  const int kbeg = bz * a.chunk;
  const int kend = min(kbeg + a.chunk, a.Lk);
  const u16* kq_base = a.qkv + a.nq * HD + g * HD;
  const u16* vq_base = a.qkv + (a.nq + a.nkv) * HD + g * HD;
#pragma unroll
  for (int it = 0; it < KIT; ++it) {
    const int item = tid + it * NT;
    const int j = min((item & 15) + 16 * (item >> 7), CH - 1), p = (item >> 4) & 7;
    int key = kbeg + j;
    key = key < kend ? key : kbeg;
    const bool win = key >= a.ws && key < a.ws + a.rows;
    if (win) {
      const u16* src = kq_base + (size_t)(key - a.ws) * a.ldq;
      R.klo[it] = ld16<false>(src + 8 * p);
      R.khi[it] = ld16<false>(src + 64 + 8 * p);
      if constexpr (WCS) {
        const float* cs = a.rope + (size_t)(key - a.ws) * 128 + 16 * p;
#pragma unroll
        for (int c = 0; c < 4; ++c) R.kcs[it][c] = *reinterpret_cast<const f32x4*>(cs + 4 * c);
      }
    } else {
      const u16* src = a.kc + key * krow + g * HD;
      R.klo[it] = *reinterpret_cast<const u32x4*>(src + 8 * p);
      R.khi[it] = *reinterpret_cast<const u32x4*>(src + 64 + 8 * p);
    }
  }
#pragma unroll
  for (int it = 0; it < VIT; ++it) {
    const int item = tid + it * NT;
    const int kq = min((item & 15) + 16 * (item >> 8), CH / 4 - 1), dc = (item >> 4) & 15;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      int key = kbeg + 4 * kq + qq;
      key = key < kend ? key : kbeg;
      const bool win = key >= a.ws && key < a.ws + a.rows;
      if (win) {
        R.vv[it][qq] = ld16<false>(vq_base + (size_t)(key - a.ws) * a.ldq + 8 * dc);
      } else {
        R.vv[it][qq] = *reinterpret_cast<const u32x4*>(a.vc + key * krow + g * HD + 8 * dc);
      }
    }
  }
}

template <int DT, int QPW, int KH, int CH, int MASK, bool WCS = false>
__device__ __forceinline__ void attn_chunk_compute(const AttnP& a, int bx, int by, int bz, unsigned char* smem,
                                                   AttnChunkRegs<QPW, KH, CH, WCS>& R, int tid) {
  typedef AttnChunkRegs<QPW, KH, CH, WCS> Regs;
  constexpr int NT = Regs::NT, KIT = Regs::KIT, VIT = Regs::VIT;
  constexpr int VLDC = CH + 8;                        // u16 stride of a transposed V row
  constexpr int DT16 = HD / 16;
  static_assert(CH % (32 * KH) == 0, "each key part must be whole 32-key blocks");
  u16* kbuf = reinterpret_cast<u16*>(smem);           // [CH][KLD]
  u16* vbuf = kbuf + CH * KLD;                        // [HD][VLDC]
  u32x4 (&klo)[KIT] = R.klo;
  u32x4 (&khi)[KIT] = R.khi;
  u32x4 (&vv)[VIT][4] = R.vv;

  const int lane = tid & 63, w = tid >> 6;
  const int qw = w % QPW, kh = w / QPW;
  const int lr = lane & 15, lg = lane >> 4;
  const int g = by, c = bz;
  const int grp = a.nq / a.nkv, QR = grp * a.rows, QT = (QR + 15) / 16;
  const int qt = bx * QPW + qw;
  const bool tile_ok = qt < QT;
  const size_t krow = (size_t)a.nkv * HD;
  const int kbeg = c * a.chunk;
  const int kend = min(kbeg + a.chunk, a.Lk);
  const bool writer = bx == 0;

  // this lane's query row (qi = 16 qt + lr), RoPE'd in registers while the chunk is in flight by the
  // first key part's wave of the tile, which leaves the fragments in LDS for the other key parts
  const int qi = qt * 16 + lr;
  const bool qvalid = tile_ok && qi < QR;
  const int hh = qvalid ? qi / a.rows : 0;
  const int r = qvalid ? qi - hh * a.rows : 0;
  // (a batched call runs three or more workgroup rounds: it skips the sharing, whose 16 KB of LDS would
  // keep a second workgroup off each compute unit, and every wave loads its queries itself)
  u32x4 qf[4] = {R.qf[0], R.qf[1], R.qf[2], R.qf[3]};  // requested by attn_chunk_qload
  u32x4* qbuf = reinterpret_cast<u32x4*>(vbuf + HD * VLDC);  // [QPW][4][64] (KH > 1)
  const bool qshare = KH > 1 && a.nseq <= 1;
  if (!qshare || kh == 0) {
    if (a.rope != nullptr) {
      rope_pairs<DT>(qf[0], qf[2], R.qcs[0]);
      rope_pairs<DT>(qf[1], qf[3], R.qcs[1]);
    }
    if (qshare) {
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) qbuf[(qw * 4 + ds) * 64 + lane] = qf[ds];
    }
  }
  const int qpos_blk = MASK == 1 ? (a.q_pos0 + r) / a.block : 0;
  const float* brow = MASK == 2 ? a.bias + (long long)r * a.bias_ld : nullptr;
  const float c2 = a.scale * LOG2E;

  // ---- stage: K rows (window rows RoPE'd and appended to the cache), V transposed ----
#pragma unroll
  for (int it = 0; it < KIT; ++it) {
    const int item = tid + it * NT;
    if (item >= CH * 8) break;
    const int j = (item & 15) + 16 * (item >> 7), p = (item >> 4) & 7;
    const int key = kbeg + j;
    u32x4 lo = klo[it], hi = khi[it];
    if (key >= kend) {
      lo = hi = u32x4{0u, 0u, 0u, 0u};
    } else if (key >= a.ws && key < a.ws + a.rows) {
      if constexpr (WCS) rope_pairs<DT>(lo, hi, R.kcs[it]);
      else rope_tab<DT>(lo, hi, a.rope + (size_t)(key - a.ws) * 128 + 16 * p);
      if (writer) {
        u16* dst = a.kc + key * krow + g * HD;
        *reinterpret_cast<u32x4*>(dst + 8 * p) = lo;
        *reinterpret_cast<u32x4*>(dst + 64 + 8 * p) = hi;
      }
    }
    *reinterpret_cast<u32x4*>(kbuf + j * KLD + 8 * p) = lo;
    *reinterpret_cast<u32x4*>(kbuf + j * KLD + 64 + 8 * p) = hi;
  }
#pragma unroll
  for (int it = 0; it < VIT; ++it) {
    const int item = tid + it * NT;
    if (item >= (CH / 4) * 16) break;
    const int kq = (item & 15) + 16 * (item >> 8), dc = (item >> 4) & 15;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int key = kbeg + 4 * kq + qq;
      if (key >= kend) {
        vv[it][qq] = u32x4{0u, 0u, 0u, 0u};
      } else if (writer && key >= a.ws && key < a.ws + a.rows) {
        *reinterpret_cast<u32x4*>(a.vc + key * krow + g * HD + 8 * dc) = vv[it][qq];
      }
    }
    // dim 8 dc + e of the quad's four keys, packed key-major into one 8-byte word (byte permutes:
    // low halves select bytes 0-1 of each word, high halves bytes 2-3)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
      const uint32_t w01 = __builtin_amdgcn_perm(vv[it][1][e >> 1], vv[it][0][e >> 1], sel);
      const uint32_t w23 = __builtin_amdgcn_perm(vv[it][3][e >> 1], vv[it][2][e >> 1], sel);
      *reinterpret_cast<u32x2*>(vbuf + (8 * dc + e) * VLDC + 4 * kq) = u32x2{w01, w23};
    }
  }
  __syncthreads();
  if (qshare && kh > 0) {
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) qf[ds] = qbuf[(qw * 4 + ds) * 64 + lane];
  }

  // ---- scores and P.V over this wave's key part ----
  // lane (lr, lg) holds S^T[key kb + 16 kt + 4 lg + i][query lr] and O^T[dim 16 dt + 4 lg + i][query lr]
  float m_run = -INFINITY, l_run = 0.f;
  f32x4 o[DT16];
#pragma unroll
  for (int dt = 0; dt < DT16; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  constexpr int KPW = CH / KH;  // keys per wave
  if (tile_ok) {
    for (int b = 0; b < KPW / 32; ++b) {
      const int kl = kh * KPW + 32 * b;  // chunk-local first key of the block
      const int kb = kbeg + kl;
      if (kb >= kend) break;
      f32x4 s[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
        const u16* kp = kbuf + (kl + 16 * kt + lr) * KLD + 8 * lg;
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) s[kt] = mfma16<DT>(*reinterpret_cast<const u32x4*>(kp + 32 * ds), qf[ds], s[kt]);
      }
      float mx = -INFINITY;
      if (MASK == 0 && kb + 32 <= kend) {  // a whole block of keys: no per-key test
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            s[kt][i] *= c2;
            mx = fmaxf(mx, s[kt][i]);
          }
      } else {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kb + 16 * kt + 4 * lg + i;
            float v = s[kt][i] * c2;
            if (key >= kend) {
              v = -INFINITY;
            } else if constexpr (MASK == 1) {
              if (qpos_blk < key / a.block) v = -INFINITY;
            } else if constexpr (MASK == 2) {
              v += brow[key] * LOG2E;
            }
            s[kt][i] = v;
            mx = fmaxf(mx, v);
          }
      }
      mx = rows_max(mx);
      const float m_new = fmaxf(m_run, mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      float ps = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pe = __builtin_amdgcn_exp2f(s[kt][i] - m_use);
          s[kt][i] = pe;
          ps += pe;
        }
      ps = rows_sum(ps);
      l_run = l_run * alpha + ps;
      m_run = m_new;
      // P^T as the B operand: k slot 8 lg + e holds key 4 lg + e (e < 4) or 16 + 4 lg + e - 4; the V^T
      // fragment (A operand) reads the same keys
      const u32x4 pb = {pack2(from_f32<DT>(s[0][0]), from_f32<DT>(s[0][1])),
                        pack2(from_f32<DT>(s[0][2]), from_f32<DT>(s[0][3])),
                        pack2(from_f32<DT>(s[1][0]), from_f32<DT>(s[1][1])),
                        pack2(from_f32<DT>(s[1][2]), from_f32<DT>(s[1][3]))};
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt) {
        const u16* vrow = vbuf + (16 * dt + lr) * VLDC + kl + 4 * lg;
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 16);
        o[dt] = mfma16<DT>(u32x4{lo[0], lo[1], hi[0], hi[1]}, pb, o[dt] * alpha);
      }
    }
  }

  // ---- merge the key parts in LDS (fixed order kh = 0, 1, ...); wave kh = 0 keeps the result ----
  __syncthreads();
  float Mq, Lq;
  {
    float* cm = reinterpret_cast<float*>(smem);
    float* cl = cm + KH * QPW * 16;
    f32x4* co = reinterpret_cast<f32x4*>(cl + KH * QPW * 16);
    if (lg == 0) {
      cm[(kh * QPW + qw) * 16 + lr] = m_run;
      cl[(kh * QPW + qw) * 16 + lr] = l_run;
    }
    if (KH > 1 && kh > 0) {
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt) co[(((kh - 1) * QPW + qw) * DT16 + dt) * 64 + lane] = o[dt];
    }
    __syncthreads();
    if (kh == 0) {
      float M = -INFINITY;
      for (int k = 0; k < KH; ++k) M = fmaxf(M, cm[(k * QPW + qw) * 16 + lr]);
      const float Mu = M == -INFINITY ? 0.f : M;
      float L = 0.f;
      for (int k = 0; k < KH; ++k) L += cl[(k * QPW + qw) * 16 + lr] * __builtin_amdgcn_exp2f(cm[(k * QPW + qw) * 16 + lr] - Mu);
      const float f0 = __builtin_amdgcn_exp2f(cm[qw * 16 + lr] - Mu);
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt) o[dt] *= f0;
      for (int k = 1; k < KH; ++k) {
        const float fk = __builtin_amdgcn_exp2f(cm[(k * QPW + qw) * 16 + lr] - Mu);
#pragma unroll
        for (int dt = 0; dt < DT16; ++dt) o[dt] += co[(((k - 1) * QPW + qw) * DT16 + dt) * 64 + lane] * fk;
      }
      Mq = M;
      Lq = L;
    }
  }

  // lane output: query row qi (head hh, row r), dims 16 dt + 4 lg .. + 3
  auto store4 = [&](int dt, f32x4 v) {
    u16* dst = out_at(a, r, (g * grp + hh) * HD + 16 * dt + 4 * lg);
    st8<false>(dst, u32x2{pack2(from_f32<DT>(v[0]), from_f32<DT>(v[1])), pack2(from_f32<DT>(v[2]), from_f32<DT>(v[3]))});
  };
  if (a.S == 1) {
    if (kh == 0 && qvalid) {
      const float inv = 1.0f / Lq;
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt) store4(dt, o[dt] * inv);
    }
    return;
  }

  // ---- key splits: the partial of (g, qt, c): O^T as f32x4 [HD / 16][64 lanes], then (m, l) of each of
  // the tile's 16 queries; attn_merge_kernel combines them ----
  if (kh == 0 && tile_ok) {
    float* pp = a.part + ((size_t)(g * QT + qt) * a.S + c) * PSZ;
#pragma unroll
    for (int dt = 0; dt < DT16; ++dt) stf4<false>(reinterpret_cast<f32x4*>(pp) + dt * 64 + lane, o[dt]);
    if (lg == 0) stf2<false>(pp + 16 * HD + 2 * lr, f32x2_t{Mq, Lq});
  }
}

template <int DT, int QPW, int KH, int CH, int MASK>
__device__ __forceinline__ void attn_chunk_body(const AttnP& a, int bx, int by, int bz, unsigned char* smem) {
  AttnChunkRegs<QPW, KH, CH, true> R;
  attn_chunk_qload<QPW, KH, CH, true>(a, bx, by, R, threadIdx.x);
  attn_chunk_load<QPW, KH, CH, true>(a, by, bz, R, threadIdx.x);
  attn_chunk_compute<DT, QPW, KH, CH, MASK, true>(a, bx, by, bz, smem, R, threadIdx.x);
}

// Batched call: the view of sequence b (its rows, cache, window and split partials) in a, a copy of the
// kernel argument p.  The per-sequence tables are read from p itself: indexing them in the copy would
// keep the whole copy in scratch memory.
__device__ __forceinline__ void seq_view(AttnP& a, const AttnP& p, int b) {
  const int QT = ((p.nq / p.nkv) * p.rows + 15) / 16;
  a.qkv = p.qkv + (size_t)b * p.rows * p.ldq;
  a.rope = p.rope + (size_t)b * p.rows * 128;
  a.out = p.out + (size_t)b * p.rows * p.nq * HD;
  a.kc = p.kc + b * p.seq_stride;
  a.vc = p.vc + b * p.seq_stride;
  a.ws = p.seq_ws[b];
  a.Lk = p.seq_lk[b];
  a.part = p.part + (size_t)b * p.nkv * QT * p.S * PSZ;
}

// One sequence: a 1-D grid in XCD-aware order.  The qg workgroups that read one (kv head, key chunk)
// pair -- one per query-tile group -- get linear indices 8 apart, so they run on one XCD (workgroup i is
// placed on XCD i % 8) and share its L2: the chunk's K/V comes from HBM once instead of once per group.
// Linear index i: XCD slot i % 8, round i / 8; pair = (round / qg) x 8 + slot (kv head pair % nkv, chunk
// pair / nkv), query-tile group round % qg.  Indices past the last pair have nothing to do.
// Batched calls: gridDim.x = query-tile groups x sequences (sequence-major), y = kv heads, z = chunks.
// MASK is the launch's AttnP::mask.
__host__ __device__ __forceinline__ int attn_chunk_grid_1seq(int qg, int nkv, int S) {
  return (nkv * S + 7) / 8 * 8 * qg;
}

template <int DT, int QPW, int KH, int CH, int MASK>
__global__ __launch_bounds__(64 * QPW * KH) void attn_chunk_kernel(AttnP p) {
  extern __shared__ __align__(16) unsigned char smem[];
  if (p.nseq <= 1) {
    const int QT = ((p.nq / p.nkv) * p.rows + 15) / 16, qg = (QT + QPW - 1) / QPW;
    const int i = blockIdx.x, round = i >> 3;
    const int pair = (round / qg) * 8 + (i & 7), x = round % qg;
    if (pair >= p.nkv * p.S) return;
    attn_chunk_body<DT, QPW, KH, CH, MASK>(p, x, pair % p.nkv, pair / p.nkv, smem);
    return;
  }
  const int qg = (int)gridDim.x / p.nseq, b = (int)blockIdx.x / qg;
  AttnP a = p;
  seq_view(a, p, b);
  if ((int)blockIdx.z * a.chunk >= a.Lk) return;  // past this sequence's keys: the merge skips it
  attn_chunk_body<DT, QPW, KH, CH, MASK>(a, (int)blockIdx.x - b * qg, blockIdx.y, blockIdx.z, smem);
}

// Merge of the key splits: one wave per (kv head g, query tile qt, 16-dim slice dt).  The split weights
// exp(m_c - M) depend only on the query, so each lane computes them once for its query lr; the split
// partials are added in split order.
// Splits at or past ceil(Lk / chunk) (a shorter sequence of a batched call) hold nothing and are skipped.
// SR: splits held in registers at once (two loads each), so that up to SR splits cost one round trip.
template <int DT, int SR = 24>
__device__ __forceinline__ void attn_merge_wave(const AttnP& a, int dt, int qt, int g, int lane) {
  constexpr int SB = 8;   // batch of the two-pass loop for more splits
  const int lr = lane & 15, lg = lane >> 4;
  const int grp = a.nq / a.nkv, QR = grp * a.rows, QT = (QR + 15) / 16;
  const int S = min(a.S, (a.Lk + a.chunk - 1) / a.chunk);  // splits that hold keys
  const float* pt = a.part + (size_t)(g * QT + qt) * a.S * PSZ;
  // O^T fragment and (m, l) of this lane's query in split q
  auto ld_o = [&](int q) -> f32x4 {
    return ldf4<false>(reinterpret_cast<const f32x4*>(pt + (size_t)q * PSZ) + dt * 64 + lane);
  };
  auto ld_ml = [&](int q) -> f32x2_t { return ldf2<false>(pt + (size_t)q * PSZ + 16 * HD + 2 * lr); };
  float M = -INFINITY, L = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (S <= SR) {
    f32x4 ov[SR];
    f32x2_t ml[SR];  // (m, l) of this lane's query
#pragma unroll
    for (int q = 0; q < SR; ++q) {
      ov[q] = ld_o(min(q, S - 1));
      ml[q] = ld_ml(min(q, S - 1));
    }
    // keep every load above issued before the first use (the scheduler would otherwise sink the O loads
    // next to their uses and pay one round trip per pair)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < SR; ++q) M = fmaxf(M, ml[q][0]);
    const float Mu = M == -INFINITY ? 0.f : M;
#pragma unroll
    for (int q = 0; q < SR; ++q) {
      const float e = q < S ? __builtin_amdgcn_exp2f(ml[q][0] - Mu) : 0.f;
      L += ml[q][1] * e;
      acc += ov[q] * e;
    }
  } else {
    for (int s0 = 0; s0 < S; s0 += SB) {
      f32x2_t mv[SB];
#pragma unroll
      for (int q = 0; q < SB; ++q) mv[q] = ld_ml(min(s0 + q, S - 1));
#pragma unroll
      for (int q = 0; q < SB; ++q) M = fmaxf(M, mv[q][0]);
    }
    const float Mu = M == -INFINITY ? 0.f : M;
    for (int s0 = 0; s0 < S; s0 += SB) {
      f32x4 ov[SB];
      f32x2_t mv[SB];
#pragma unroll
      for (int q = 0; q < SB; ++q) {
        ov[q] = ld_o(min(s0 + q, S - 1));
        mv[q] = ld_ml(min(s0 + q, S - 1));
      }
#pragma unroll
      for (int q = 0; q < SB; ++q) {
        const float e = s0 + q < S ? __builtin_amdgcn_exp2f(mv[q][0] - Mu) : 0.f;
        L += mv[q][1] * e;
        acc += ov[q] * e;
      }
    }
  }
  const int qi = qt * 16 + lr;
  if (qi < QR) {
    const int h = qi / a.rows, r = qi - h * a.rows;
    const float inv = 1.0f / L;
    u16* dst = out_at(a, r, (g * grp + h) * HD + 16 * dt + 4 * lg);
    st8<false>(dst, u32x2{pack2(from_f32<DT>(acc[0] * inv), from_f32<DT>(acc[1] * inv)),
                          pack2(from_f32<DT>(acc[2] * inv), from_f32<DT>(acc[3] * inv))});
  }
}

// gridDim.z = kv heads x sequences (sequence-major).  SR: the splits one round trip covers (the launcher
// picks 24 or, for more splits, 40; a one-wave workgroup can spend the registers).
template <int DT, int SR>
__global__ __launch_bounds__(64) void attn_merge_kernel(AttnP p) {
  if (p.nseq <= 1) {
    attn_merge_wave<DT, SR>(p, blockIdx.x, blockIdx.y, blockIdx.z, threadIdx.x);
    return;
  }
  const int b = (int)blockIdx.z / p.nkv;
  AttnP a = p;
  seq_view(a, p, b);
  attn_merge_wave<DT, SR>(a, blockIdx.x, blockIdx.y, (int)blockIdx.z - b * p.nkv, threadIdx.x);
}


// ---- long row blocks (prefill, stateless forward): RoPE + KV append pass, then a flash-style kernel --
// rope_kv_kernel: one workgroup per row r.  q heads are RoPE'd into out (the attention output buffer,
// [rows][nq * 128]: the prefill kernel reads each query from there before it writes that query's
// output), k heads are RoPE'd and v copied into the cache rows ws + r (the KV append of
// fast_dllm.attn_inplace, runtime.py:51-60).  Same RoPE arithmetic as the chunk kernels.
// Batched calls (nseq > 1): workgroup b rows + r is row r of sequence b, in that sequence's view.
template <int DT>
__device__ __forceinline__ void rope_kv_row(const AttnP& a, int r) {
  const u16* src = a.qkv + (size_t)r * a.ldq;
  const float* cs = a.rope + (size_t)r * 128;
  const size_t krow = (size_t)a.nkv * HD;
  const int nrope = (a.nq + a.nkv) * 8;  // (head, rotation-pair chunk) items
  for (int item = threadIdx.x; item < nrope + a.nkv * 16; item += 128) {
    if (item < nrope) {
      const int hd = item >> 3, p = item & 7;
      const u16* hs = src + hd * HD;
      u32x4 lo = *reinterpret_cast<const u32x4*>(hs + 8 * p);
      u32x4 hi = *reinterpret_cast<const u32x4*>(hs + 64 + 8 * p);
      rope_tab<DT>(lo, hi, cs + 16 * p);
      u16* dst = hd < a.nq ? a.out + (size_t)r * a.nq * HD + hd * HD
                           : a.kc + (size_t)(a.ws + r) * krow + (hd - a.nq) * HD;
      *reinterpret_cast<u32x4*>(dst + 8 * p) = lo;
      *reinterpret_cast<u32x4*>(dst + 64 + 8 * p) = hi;
    } else {
      const int it = item - nrope, g = it >> 4, c = it & 15;
      *reinterpret_cast<u32x4*>(a.vc + (size_t)(a.ws + r) * krow + g * HD + 8 * c) =
          *reinterpret_cast<const u32x4*>(src + (a.nq + a.nkv + g) * HD + 8 * c);
    }
  }
}
template <int DT>
__global__ __launch_bounds__(128) void rope_kv_kernel(AttnP p) {
  if (p.nseq <= 1) {
    rope_kv_row<DT>(p, blockIdx.x);
    return;
  }
  const int b = (int)blockIdx.x / p.rows;
  AttnP a = p;
  seq_view(a, p, b);
  rope_kv_row<DT>(a, (int)blockIdx.x - b * p.rows);
}

// attn_prefill_kernel: workgroup (query block of 32 rows, head subset hg of kv head g) with NWQ waves x
// TQ query tiles (2 tiles per head: rows q0 .. q0 + 15 and q0 + 16 .. q0 + 31 of head hh).  The kv head's
// keys stream through LDS in blocks of 64 (K row-major, V transposed), double-buffered: the next block
// is loaded into registers while this one is multiplied, so every K/V row is read once per workgroup
// for all of its query tiles.  Scores in fp32 on MFMA, online softmax in base 2 with the scale folded
// in (p = 2^(s * scale * log2 e - m)), P rounded to the model dtype for P.V, fp32 accumulation; the
// precision order of the chunk kernels.  MASK 1 (block-causal, cuda.py:148-177) reduces to a key
// bound per query: keys below ((q_pos0 + r) / block + 1) * block.  Query blocks are dealt heaviest
// (latest) first.  Queries come from out (rope_kv_kernel) and results go back to the same places.
template <int DT, int MASK, int TQ, int NWQ>
__global__ __launch_bounds__(64 * NWQ) void attn_prefill_kernel(AttnP a, int hpw) {
  constexpr int KBP = 64;          // keys per block
  constexpr int KLDP = HD + 8;     // u16 stride of a K row
  constexpr int VLDP = KBP + 8;    // u16 stride of a V^T row
  constexpr int NT = 64 * NWQ;
  constexpr int KIT = KBP * 16 / NT;       // 16-byte K chunks per thread per block
  constexpr int VIT = (KBP / 4) * 16 / NT; // (key quad, dim chunk) V items per thread per block
  static_assert(KIT * NT == KBP * 16 && VIT * NT == (KBP / 4) * 16, "whole staging rounds");
  static_assert(MASK == 0 || MASK == 1, "explicit biases take attn_kernel");
  constexpr int DT16 = HD / 16;
  extern __shared__ __align__(16) unsigned char smem[];
  // buffer b: K at element b * BUFE, V^T after it.  Offsets from the shared array itself (not pointers
  // picked from a local array), so that every access stays a direct LDS access instead of a flat one.
  constexpr int BUFE = KBP * KLDP + HD * VLDP;
  u16* const lds16 = reinterpret_cast<u16*>(smem);

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int grp = a.nq / a.nkv, nhg = grp / hpw;
  const int nqb = (a.rows + 31) / 32;
  const int qb = nqb - 1 - (int)blockIdx.x / nhg, hg = (int)blockIdx.x % nhg;
  const int g = blockIdx.y;
  const int q0 = qb * 32, rlast = a.rows - 1;
  const size_t krow = (size_t)a.nkv * HD;
  const u16* kc = a.kc + g * HD;
  const u16* vc = a.vc + g * HD;
  const float c2 = a.scale * LOG2E;

  // the keys this workgroup needs: up to its last query's bound
  auto kend_of = [&](int r) {
    if constexpr (MASK == 1) return min(a.Lk, ((a.q_pos0 + r) / a.block + 1) * a.block);
    return a.Lk;
  };
  const int kend_wg = kend_of(min(q0 + 31, rlast));
  const int nkb = (kend_wg + KBP - 1) / KBP;

  // this wave's query tiles: tile t = w TQ + i -> head hg hpw + t / 2, rows q0 + 16 (t % 2) + lr
  u32x4 qf[TQ][4];
  int kend_q[TQ];
  bool tvalid[TQ];
  const u16* qsrc = a.out;
#pragma unroll
  for (int i = 0; i < TQ; ++i) {
    const int t = w * TQ + i;
    tvalid[i] = t < 2 * hpw && q0 + 16 * (t % 2) <= rlast;
    const int hh = hg * hpw + min(t, 2 * hpw - 1) / 2;
    const int r = min(q0 + 16 * (t % 2) + lr, rlast);
    kend_q[i] = kend_of(r);
    const u16* qp = qsrc + (size_t)r * a.nq * HD + (g * grp + hh) * HD + 8 * lg;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) qf[i][ds] = *reinterpret_cast<const u32x4*>(qp + 32 * ds);
  }

  // staging maps (conflict-free LDS stores): K item -> key j, 16-byte chunk c; V item -> key quad kq, dim chunk dc
  u32x4 kr[KIT], vr[VIT][4];
  auto load = [&](int kb) {
    const int k0 = kb * KBP;
#pragma unroll
    for (int it = 0; it < KIT; ++it) {
      const int item = threadIdx.x + it * NT;
      const int j = (item & 15) + 16 * (item >> 8), c = (item >> 4) & 15;
      const int key = min(k0 + j, kend_wg - 1);
      kr[it] = *reinterpret_cast<const u32x4*>(kc + (size_t)key * krow + 8 * c);
    }
#pragma unroll
    for (int it = 0; it < VIT; ++it) {
      const int item = threadIdx.x + it * NT;
      const int kq = item & 15, dc = item >> 4;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int key = min(k0 + 4 * kq + qq, kend_wg - 1);
        vr[it][qq] = *reinterpret_cast<const u32x4*>(vc + (size_t)key * krow + 8 * dc);
      }
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int it = 0; it < KIT; ++it) {
      const int item = threadIdx.x + it * NT;
      const int j = (item & 15) + 16 * (item >> 8), c = (item >> 4) & 15;
      *reinterpret_cast<u32x4*>(lds16 + buf * BUFE + j * KLDP + 8 * c) = kr[it];
    }
#pragma unroll
    for (int it = 0; it < VIT; ++it) {
      const int item = threadIdx.x + it * NT;
      const int kq = item & 15, dc = item >> 4;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        const uint32_t w01 = __builtin_amdgcn_perm(vr[it][1][e >> 1], vr[it][0][e >> 1], sel);
        const uint32_t w23 = __builtin_amdgcn_perm(vr[it][3][e >> 1], vr[it][2][e >> 1], sel);
        *reinterpret_cast<u32x2*>(lds16 + buf * BUFE + KBP * KLDP + (8 * dc + e) * VLDP + 4 * kq) = u32x2{w01, w23};
      }
    }
  };

  float m_run[TQ], l_run[TQ];
  f32x4 o[TQ][DT16];
#pragma unroll
  for (int i = 0; i < TQ; ++i) {
    m_run[i] = -INFINITY;
    l_run[i] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT16; ++dt) o[i][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  load(0);
  stage(0);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    load(min(kb + 1, nkb - 1));
    const u16* kbuf = lds16 + buf * BUFE;
    const u16* vbuf = kbuf + KBP * KLDP;
    const int k0 = kb * KBP;
#pragma unroll
    for (int i = 0; i < TQ; ++i) {
      if (!tvalid[i]) continue;
      // S^T = K Q^T: lane holds S^T[key k0 + 16 kt + 4 lg + e][query lr]
      f32x4 s[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
        const u16* kp = kbuf + (16 * kt + lr) * KLDP + 8 * lg;
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) s[kt] = mfma16<DT>(*reinterpret_cast<const u32x4*>(kp + 32 * ds), qf[i][ds], s[kt]);
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = k0 + 16 * kt + 4 * lg + e;
          const float v = key < kend_q[i] ? s[kt][e] * c2 : -INFINITY;
          s[kt][e] = v;
          mx = fmaxf(mx, v);
        }
      mx = rows_max(mx);
      const float m_new = fmaxf(m_run[i], mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run[i] - m_use);
      float ps = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pe = __builtin_amdgcn_exp2f(s[kt][e] - m_use);
          s[kt][e] = pe;
          ps += pe;
        }
      ps = rows_sum(ps);
      l_run[i] = l_run[i] * alpha + ps;
      m_run[i] = m_new;
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt) o[i][dt] *= alpha;
      // O^T += V^T P^T over the block's two 32-key k steps (k slot 8 lg + e: key 4 lg + e, then 16 + 4 lg + e - 4)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const u32x4 pb = {pack2(from_f32<DT>(s[2 * ks][0]), from_f32<DT>(s[2 * ks][1])),
                          pack2(from_f32<DT>(s[2 * ks][2]), from_f32<DT>(s[2 * ks][3])),
                          pack2(from_f32<DT>(s[2 * ks + 1][0]), from_f32<DT>(s[2 * ks + 1][1])),
                          pack2(from_f32<DT>(s[2 * ks + 1][2]), from_f32<DT>(s[2 * ks + 1][3]))};
#pragma unroll
        for (int dt = 0; dt < DT16; ++dt) {
          const u16* vrow = vbuf + (16 * dt + lr) * VLDP + 32 * ks + 4 * lg;
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 16);
          o[i][dt] = mfma16<DT>(u32x4{lo[0], lo[1], hi[0], hi[1]}, pb, o[i][dt]);
        }
      }
    }
    stage(buf ^ 1);
    __syncthreads();
  }

  // lane output: query row r of tile i, dims 16 dt + 4 lg .. + 3
#pragma unroll
  for (int i = 0; i < TQ; ++i) {
    const int t = w * TQ + i;
    const int r = q0 + 16 * (t % 2) + lr;
    if (!tvalid[i] || r > rlast) continue;
    const int hh = hg * hpw + t / 2;
    const float inv = 1.0f / l_run[i];
    u16* dst = a.out + (size_t)r * a.nq * HD + (g * grp + hh) * HD + 4 * lg;
#pragma unroll
    for (int dt = 0; dt < DT16; ++dt)
      *reinterpret_cast<u32x2*>(dst + 16 * dt) =
          u32x2{pack2(from_f32<DT>(o[i][dt][0] * inv), from_f32<DT>(o[i][dt][1] * inv)),
                pack2(from_f32<DT>(o[i][dt][2] * inv), from_f32<DT>(o[i][dt][3] * inv))};
  }
}

// attn_prefill_pair_kernel: the long-prefill form of attn_prefill_kernel.  Workgroup (p, g) owns kv head
// g and the pair of 32-row query blocks nqb - 1 - p and p: under the block-causal mask their key ranges
// add up to the same number of 64-key blocks for every pair, so with one workgroup per compute unit all
// finish together (one block per workgroup, as in attn_prefill_kernel, leaves the longest query block
// alone on its compute unit at the end).  The workgroup's 4 TQ query tiles (TQ per wave) are tiles
// 4 TQ z .. of the kv head's 2 grp (blockIdx.z = z): with TQ = grp / 2 all heads of the kv head are in one
// workgroup, so each K/V block fetched serves all of them; shorter prefills, with too few pairs to fill
// the chip, split the heads over 2 grp / (4 TQ) workgroups.  A wave reads each K or V fragment from LDS
// once for its TQ tiles.  Per query the key blocks, their order and every rounding are
// those of attn_prefill_kernel, so the results are the same bits.
//
// The work is a list of tasks t = (query block, key block): the first block's key blocks, then the
// second's.  Task t's K and V rows go from global memory straight into LDS buffer t % R (R = D + 1) by
// the gfx950 global-to-LDS copy, D tasks ahead, so no registers hold data in flight and no VALU work
// stages it.  Both are stored row-major (a 256-byte row per key) with the 16-byte chunk c of row r at
// slot c ^ (r % 16): the copy's lanes fetch their chunks in that order, the K fragment reads (16 rows,
// one chunk each) then hit 16 different slots, and so do the V reads.  V^T fragments come from the
// transposing LDS read (ds_read_b64_tr_b16): within each 16-lane group, lane q supplies 4 dims of one
// key (key q / 4, dims 4 (q % 4) ..) and lane m receives dim m of the 4 keys, which is the A operand of
// O^T = V^T P^T for keys 4 lg .. 4 lg + 3 (and, from a second read, 16 + 4 lg ..): the k-slot order the
// scores already have in registers.
template <int DT, int MASK, int TQ, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void attn_prefill_pair_kernel(AttnP a) {
  constexpr int NWQ = 4, R = D + 1;
  constexpr int KBP = 64;               // keys per block (task)
  constexpr int BUFE = 2 * KBP * HD;    // u16 per buffer: K rows, then V rows
  constexpr int CPW = KBP * HD * 2 / 1024 / NWQ;  // 1 KB copies of K (and of V) per wave per task
  static_assert(MASK == 0 || MASK == 1, "explicit biases take attn_kernel");
  static_assert(D >= 1 && (D - 1) * 2 * CPW < 64, "outstanding copies fit the memory counter");
  constexpr int DT16 = HD / 16;
  extern __shared__ __align__(16) unsigned char smem[];
  u16* const lds16 = reinterpret_cast<u16*>(smem);

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int grp = a.nq / a.nkv;  // = NWQ TQ gridDim.z / 2 (the launcher checks)
  const int nqb = (a.rows + 31) / 32;
  const int p = blockIdx.x, g = blockIdx.y;
  const int tq0 = (int)blockIdx.z * NWQ * TQ;  // the workgroup's first query tile of the kv head
  const int qA = nqb - 1 - p, qB = p;  // qA == qB: the middle block of an odd count, alone
  const int rlast = a.rows - 1;
  const size_t krow = (size_t)a.nkv * HD;
  const u16* kc = a.kc + g * HD;
  const u16* vc = a.vc + g * HD;
  const float c2 = a.scale * LOG2E;

  auto kend_of = [&](int r) {
    if constexpr (MASK == 1) return min(a.Lk, ((a.q_pos0 + r) / a.block + 1) * a.block);
    return a.Lk;
  };
  auto kend_blk = [&](int qb) { return kend_of(min(qb * 32 + 31, rlast)); };
  const int keA = kend_blk(qA), keB = kend_blk(qB);
  const int nA = (keA + KBP - 1) / KBP;
  // this lane's K fragment byte offsets within a buffer: row lr, chunk lg + 4 ds (swizzled; + 4096 bytes
  // per 16-row score tile)
  uint32_t koff[4];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) koff[ds] = 2 * (lr * HD + 8 * ((lg + 4 * ds) ^ lr));
  const int T = nA + (qA == qB ? 0 : (keB + KBP - 1) / KBP);

  // ---- copies of task t (tasks past the last re-read the last) into buffer t % R: this wave's 1 KB
  // blocks d = w CPW .. + CPW - 1 of K and of V, 4 rows each; lane l fills row 4 d + l / 16, slot l % 16
  // with chunk (l % 16) ^ (row % 16) ----
  auto issue = [&](int t) __attribute__((always_inline)) {
    const int tt = min(t, T - 1);
    const int k0 = (tt < nA ? tt : tt - nA) * KBP, kend = tt < nA ? keA : keB;
    unsigned char* buf = smem + (size_t)(t % R) * BUFE * 2;
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int d = w * CPW + c, row = 4 * d + (lane >> 4);
      const int chunk = (lane & 15) ^ (row & 15);
      const size_t src = (size_t)min(k0 + row, kend - 1) * krow + 8 * chunk;
      lds_copy16(kc + src, buf + (size_t)d * 1024);
      lds_copy16(vc + src, buf + (size_t)KBP * HD * 2 + (size_t)d * 1024);
    }
  };

  // ---- the wave's query tiles of the current query block: tile w TQ + i = head (w TQ + i) / 2, rows
  // q0 + 16 ((w TQ + i) % 2) + lr ----
  u32x4 qf[TQ][4];
  int kend_q[TQ];
  int kend_min = 0;  // the block's first row's key bound, the smallest of its rows
  float m_run[TQ], l_run[TQ];
  f32x4 o[TQ][DT16];
  auto begin_block = [&](int qb) __attribute__((always_inline)) {
    const int q0 = qb * 32;
    kend_min = kend_of(q0);
#pragma unroll
    for (int i = 0; i < TQ; ++i) {
      const int t = tq0 + w * TQ + i, hh = t / 2;
      const int r = min(q0 + 16 * (t % 2) + lr, rlast);
      kend_q[i] = kend_of(r);
      const u16* qp = a.out + (size_t)r * a.nq * HD + (g * grp + hh) * HD + 8 * lg;
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) qf[i][ds] = *reinterpret_cast<const u32x4*>(qp + 32 * ds);
      // o is not cleared here: with m_run = -inf the block's first key block rescales it by
      // alpha = 2^-inf = 0 (o is always finite, and -0 + x = x)
      m_run[i] = -INFINITY;
      l_run[i] = 0.f;
    }
    // the query loads land here, once per query block: otherwise the compiler's wait before the first
    // MFMA of every key block covers them (they may be the youngest loads on the other path of the
    // branch), which waits for every copy in flight and drains the copy pipeline on each block
    wait_vmcnt<0>();
  };
  auto end_block = [&](int qb) __attribute__((always_inline)) {
    const int q0 = qb * 32;
#pragma unroll
    for (int i = 0; i < TQ; ++i) {
      const int t = tq0 + w * TQ + i, hh = t / 2;
      const int r = q0 + 16 * (t % 2) + lr;
      if (r > rlast) continue;
      const float inv = 1.0f / l_run[i];
      u16* dst = a.out + (size_t)r * a.nq * HD + (g * grp + hh) * HD + 4 * lg;
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt)
        *reinterpret_cast<u32x2*>(dst + 16 * dt) =
            u32x2{pack_f32x2<DT>(o[i][dt][0] * inv, o[i][dt][1] * inv), pack_f32x2<DT>(o[i][dt][2] * inv, o[i][dt][3] * inv)};
    }
  };

  // ---- one key block of task t against the wave's TQ tiles ----
  auto compute = [&](int t) __attribute__((always_inline)) {
    const u16* kbuf = lds16 + (size_t)(t % R) * BUFE;
    const u16* vbuf = kbuf + KBP * HD;
    const int k0 = (t < nA ? t : t - nA) * KBP;
    // S^T = K Q^T: lane holds S^T[key k0 + 16 kt + 4 lg + e][query lr]; K row 16 kt + lr, chunk lg + 4 ds.
    // The four fragments of score tile kt + 1 are requested (asm reads, one wait for the four) before tile
    // kt's MFMAs, so each wait finds them landed (the compiler's own order read one fragment, waited the
    // whole LDS latency and issued its TQ MFMAs, sixteen times per block)
    f32x4 s[TQ][4];
    const uint32_t kbb = lds_addr(kbuf);
    u32x4 kf0[4], kf1[4];
    auto rdk = [&](auto ktc, u32x4 (&f)[4]) __attribute__((always_inline)) {
      constexpr int KT = decltype(ktc)::value;
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) f[ds] = ds_read16<KT * 4096>(kbb + koff[ds]);
    };
    auto mmk = [&](int kt, const u32x4 (&f)[4]) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < TQ; ++i) s[i][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < 4; ++ds)
#pragma unroll
        for (int i = 0; i < TQ; ++i) s[i][kt] = mfma16<DT>(f[ds], qf[i][ds], s[i][kt]);
    };
    rdk(std::integral_constant<int, 0>{}, kf0);
    lds_wait(kf0);
    rdk(std::integral_constant<int, 1>{}, kf1);
    mmk(0, kf0);
    lds_wait(kf1);
    rdk(std::integral_constant<int, 2>{}, kf0);
    mmk(1, kf1);
    lds_wait(kf0);
    rdk(std::integral_constant<int, 3>{}, kf1);
    mmk(2, kf0);
    lds_wait(kf1);
    mmk(3, kf1);
    // V^T fragments of k step ks by transposing reads (ds_read_tr16: the builtin would make the compiler
    // wait for every copy in flight first): this lane supplies key 32 ks + 4 lg + lr / 4 (+ 16 for the
    // second half), dims 16 dt + 4 (lr % 4) .. + 3.  k step 0's reads are issued here and land during the
    // softmax; k step 1's during k step 0's MFMAs (both k steps' P.V after each tile's own softmax
    // measured the same, with 30 more registers)
    const uint32_t vbase = lds_addr(vbuf);
    auto rdv = [&](int ks, u32x2 (&vh)[DT16 * 2]) __attribute__((always_inline)) {
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const int row = 32 * ks + 16 * hf + 4 * lg + (lr >> 2);
          const int dim = 16 * dt + 4 * (lr & 3);
          vh[dt * 2 + hf] = ds_read_tr16(vbase + 2 * (row * HD + 8 * ((dim >> 3) ^ (row & 15)) + (dim & 7)));
        }
    };
    u32x2 vh0[DT16 * 2], vh1[DT16 * 2];
    rdv(0, vh0);
    u32x4 pb[TQ][2];
    const bool whole = k0 + KBP <= kend_min;  // no key of the block is masked for any query of the block
#pragma unroll
    for (int i = 0; i < TQ; ++i) {
      float mx = -INFINITY;
      if (whole) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s[i][kt][e] *= c2;
            mx = fmaxf(mx, s[i][kt][e]);
          }
      } else {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = k0 + 16 * kt + 4 * lg + e;
            const float v = key < kend_q[i] ? s[i][kt][e] * c2 : -INFINITY;
            s[i][kt][e] = v;
            mx = fmaxf(mx, v);
          }
      }
      mx = rows_max(mx);
      const float m_new = fmaxf(m_run[i], mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run[i] - m_use);
      float ps = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pe = __builtin_amdgcn_exp2f(s[i][kt][e] - m_use);
          s[i][kt][e] = pe;
          ps += pe;
        }
      ps = rows_sum(ps);
      l_run[i] = l_run[i] * alpha + ps;
      m_run[i] = m_new;
      // rescale only when some query's running maximum moved (alpha = 1 leaves o unchanged bit for bit);
      // past the first blocks it rarely does, and o can stay in the accumulation registers
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
        for (int dt = 0; dt < DT16; ++dt) o[i][dt] *= alpha;
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        pb[i][ks] = u32x4{pack_f32x2<DT>(s[i][2 * ks][0], s[i][2 * ks][1]),
                          pack_f32x2<DT>(s[i][2 * ks][2], s[i][2 * ks][3]),
                          pack_f32x2<DT>(s[i][2 * ks + 1][0], s[i][2 * ks + 1][1]),
                          pack_f32x2<DT>(s[i][2 * ks + 1][2], s[i][2 * ks + 1][3])};
    }
    // O^T += V^T P^T over the block's two 32-key k steps
    auto mmv = [&](int ks, const u32x2 (&vh)[DT16 * 2]) __attribute__((always_inline)) {
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt) {
        const u32x4 vf = u32x4{vh[2 * dt][0], vh[2 * dt][1], vh[2 * dt + 1][0], vh[2 * dt + 1][1]};
#pragma unroll
        for (int i = 0; i < TQ; ++i) o[i][dt] = mfma16<DT>(vf, pb[i][ks], o[i][dt]);
      }
    };
    lds_wait(vh0);
    rdv(1, vh1);
    mmv(0, vh0);
    lds_wait(vh1);
    mmv(1, vh1);
  };

  // ---- task t: wait for its copies, free buffer (t - 1) % R, issue task t + D into it, compute.
  // EXACT: the D - 1 tasks issued after task t each issued 2 CPW copies per wave, so a count wait is
  // exact (loads and stores of queries and outputs issued in between only make it wait longer); the last
  // T % D tasks, after the loop, wait for everything ----
  auto iter = [&](int t, auto exact) __attribute__((always_inline)) {
    if constexpr (decltype(exact)::value) wait_vmcnt<(D - 1) * 2 * CPW>();
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();  // every wave's copies of task t have landed; buffer (t - 1) % R is free
    __builtin_amdgcn_sched_barrier(0);
    issue(t + D);
    __builtin_amdgcn_sched_barrier(0);
    if (t == nA) begin_block(qB);
    compute(t);
    if (t == nA - 1) end_block(qA);
    else if (t == T - 1) end_block(qB);
  };

#pragma unroll
  for (int t = 0; t < D; ++t) issue(t);
#pragma unroll
  for (int i = 0; i < TQ; ++i)
#pragma unroll
    for (int dt = 0; dt < DT16; ++dt) o[i][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  begin_block(qA);
  int t0 = 0;
#pragma nounroll
  for (; t0 + D <= T; t0 += D)
    static_for<0, D>([&](auto uc) __attribute__((always_inline)) { iter(t0 + decltype(uc)::value, std::true_type{}); });
  static_for<0, D - 1>([&](auto uc) __attribute__((always_inline)) {
    if (t0 + decltype(uc)::value < T) iter(t0 + decltype(uc)::value, std::false_type{});
  });
  wait_vmcnt<0>();  // no copy may still be writing LDS when the workgroup ends
}

// attn_seq_kernel: the attention of a batched call (nseq sequences of `rows` rows each, no mask) without
// a merge launch.  Workgroup (unit u = split js of sequence b's 64-key blocks [tb, te), kv head g, group
// x of NQW query tiles) with NQW KH waves: wave w takes query tile NQW x + w % NQW of the stacked rows of
// the chunk kernels (row qi = head in group x rows + r, 16 per tile) and key part kh = w / NQW, i.e. keys
// 64 j + 64 / KH kh .. of every block j of the split (keys past Lk_b masked).  The blocks stream through
// LDS, D blocks ahead, by the global-to-LDS copy in the paired prefill kernel's layout (a 256-byte row per
// key, 16-byte chunk c of row r at slot c ^ (r % 16); V^T fragments from the transposing LDS read).
// rope_kv_kernel has already appended this call's K/V rows to the cache and put the RoPE'd queries in
// out, so every key comes from the cache and each query is read from out before its output is written
// there.  Per query and key part: one online softmax over the part's keys in order (scores in fp32, base
// 2), P rounded to the model dtype, fp32 accumulation; the KH parts are merged in LDS in part order (the
// chunk kernel's merge), then one rounding of the output.  The block loop is software-pipelined by one
// block: the scores of block t + 1 are formed while block t's softmax and P.V run (same arithmetic and
// order per block; measured 16.8 -> 16.0 us per layer on the 512-row batched step).
// A sequence of one split writes its output directly; splits merge as described at the end.
// 1-D grid in XCD-aware order: linear index i, slot i % 8, round i / 8; pair (u, g) = (round / XG) x 8 +
// slot, query group x = round % XG, so the XG workgroups that read one split's K/V run on one XCD and
// share its L2.  Indices past the last pair have nothing to do.
template <int DT, int D, int NQW, int KH>
__global__ __launch_bounds__(64 * NQW * KH) __attribute__((amdgpu_waves_per_eu(NQW * KH > 4 ? 2 : 1, NQW * KH > 4 ? 2 : 1)))
void attn_seq_kernel(AttnP p) {
  constexpr int NW = NQW * KH, R = D + 1;
  constexpr int KBP = 64;                        // keys per block
  constexpr int KPP = KBP / KH;                  // keys of a block per key part
  constexpr int BUFE = 2 * KBP * HD;             // u16 per buffer: K rows, then V rows
  constexpr int CPW = KBP * HD * 2 / 1024 / NW;  // 1 KB copies of K (and of V) per wave per block
  constexpr int DT16 = HD / 16;
  constexpr int KT = KPP / 16;                   // 16-key score tiles per part
  constexpr int KS = KPP / 32;                   // 32-key P.V steps per part
  static_assert(KH == 1 || KH == 2, "one or two key parts");
  static_assert(D >= 2 && (D - 1) * 2 * CPW < 64, "two blocks in flight; outstanding copies fit the memory counter");
  static_assert((size_t)KH * NQW * (DT16 * 64 * 16 + 2 * 16 * 4) <= (size_t)R * BUFE * 2, "merge fits the buffers");
  extern __shared__ __align__(16) unsigned char smem[];

  const int grp = p.nq / p.nkv, QR = grp * p.rows, QT = (QR + 15) / 16, XG = (QT + NQW - 1) / NQW;
  const int i = blockIdx.x, round = i >> 3;
  const int pair = (round / XG) * 8 + (i & 7), x = round % XG;
  if (pair >= p.nunits * p.nkv) return;
  const int u = pair / p.nkv, g = pair - u * p.nkv;
  const int ua = p.unit_a[u], ut = p.unit_t[u];
  const int b = ua & 63, js = (ua >> 6) & 31, ns = (ua >> 11) & 31, u0 = ua >> 16;  // partials at u0 + js
  const int tb = ut & 0xffff;  // this split's key blocks [tb, tb + T)
  AttnP a = p;
  seq_view(a, p, b);

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int qw = w % NQW, kh = w / NQW;
  const int lr = lane & 15, lg = lane >> 4;
  const int Lk = a.Lk, T = (ut >> 16) - tb;
  const size_t krow = (size_t)a.nkv * HD;
  const u16* kc = a.kc + g * HD + (size_t)tb * KBP * krow;  // block t of the split: the sequence's tb + t
  const u16* vc = a.vc + g * HD + (size_t)tb * KBP * krow;
  const float c2 = a.scale * LOG2E;

  // copies of block t (blocks past the last re-read the last) into buffer t % R: this wave's 1 KB pieces
  // d = w CPW .. + CPW - 1 of K and of V, 4 rows each; lane l fills row 4 d + l / 16, slot l % 16 with
  // chunk (l % 16) ^ (row % 16); in the last block rows past Lk repeat row Lk - 1 (masked below).  The
  // lane's offsets within a block are computed once.
  int src_off[CPW];
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const int row = 4 * (w * CPW + c) + (lane >> 4);
    src_off[c] = row * (int)krow + 8 * ((lane & 15) ^ (row & 15));
  }
  const int Lks = Lk - tb * KBP;  // the sequence's keys from the split's first
  auto issue = [&](int t) __attribute__((always_inline)) {
    const int k0 = min(t, T - 1) * KBP;
    unsigned char* buf = smem + (size_t)(t % R) * BUFE * 2;
    const u16* kb = kc + (size_t)k0 * krow;
    const u16* vb = vc + (size_t)k0 * krow;
    if (k0 + KBP <= Lks) {
#pragma unroll
      for (int c = 0; c < CPW; ++c) {
        const int d = w * CPW + c;
        lds_copy16(kb + src_off[c], buf + (size_t)d * 1024);
        lds_copy16(vb + src_off[c], buf + (size_t)KBP * HD * 2 + (size_t)d * 1024);
      }
    } else {
#pragma unroll
      for (int c = 0; c < CPW; ++c) {
        const int d = w * CPW + c, row = 4 * d + (lane >> 4);
        const int src = (min(k0 + row, Lks - 1) - k0) * (int)krow + 8 * ((lane & 15) ^ (row & 15));
        lds_copy16(kb + src, buf + (size_t)d * 1024);
        lds_copy16(vb + src, buf + (size_t)KBP * HD * 2 + (size_t)d * 1024);
      }
    }
  };
  // this lane's query: qi = 16 tile + lr (lanes past the stacked rows read row 0 and store nothing),
  // requested before the key blocks so that block 0's wait covers it
  const int tile = x * NQW + qw;
  const int qi = tile * 16 + lr;
  const bool qvalid = tile < QT && qi < QR;
  const int hh = qvalid ? qi / a.rows : 0;
  const int r = qvalid ? qi - hh * a.rows : 0;
  u32x4 qf[4];
  {
    const u16* qp = a.out + (size_t)r * a.nq * HD + (g * grp + hh) * HD + 8 * lg;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) qf[ds] = *reinterpret_cast<const u32x4*>(qp + 32 * ds);
  }
#pragma unroll
  for (int t = 0; t < D; ++t) issue(t);
  float m_run = -INFINITY, l_run = 0.f;
  f32x4 o[DT16];
#pragma unroll
  for (int dt = 0; dt < DT16; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // LDS byte offsets of this lane's fragments within a buffer: K row kp0 + lr, chunk lg + 4 ds (+ 16 rows
  // = 4096 bytes per score tile kt); V^T read at key kp0 + 4 lg + lr / 4, dims 16 dt + 4 (lr % 4) .. + 3
  // (+ 16 keys = 4096 bytes for the second half of a 32-key step, + 8192 per step); swizzled chunks
  const int kp0 = kh * KPP;  // the part's first key within a block
  uint32_t koff[4], voff[DT16];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) koff[ds] = 2 * ((kp0 + lr) * HD + 8 * ((lg + 4 * ds) ^ lr));
#pragma unroll
  for (int dt = 0; dt < DT16; ++dt) {
    const int row = kp0 + 4 * lg + (lr >> 2), dim = 16 * dt + 4 * (lr & 3);
    voff[dt] = 2 * (KBP * HD + row * HD + 8 * ((dim >> 3) ^ (row & 15)) + (dim & 7));
  }
  const uint32_t lds0 = lds_addr(smem);

  // this wave's part of one key block against its query tile
  // Block t in three parts, so that one block's scores overlap the previous block's softmax and P.V:
  // read_k / read_v issue this lane's LDS fragment reads (no wait), qk forms S^T = K Q^T once the K
  // fragments are in, soft turns block t's scores into P (the online softmax), pv adds V^T P^T.
  // S^T: lane holds S^T[key k0 + 16 kt + 4 lg + e][query lr]; V^T read by the transposing read (this lane
  // supplies key kp0 + 32 ks + 4 lg + lr / 4 (+ 16 for the second half), dims 16 dt + 4 (lr % 4) .. + 3).
  auto read_k = [&](int t, u32x4 (&kf)[KT * 4]) __attribute__((always_inline)) {
    const uint32_t bufb = lds0 + (uint32_t)(t % R) * (BUFE * 2);
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      const uint32_t ka = bufb + koff[ds];
      static_for<0, KT>([&](auto kt) __attribute__((always_inline)) {
        kf[decltype(kt)::value * 4 + ds] = ds_read16<decltype(kt)::value * 4096>(ka);
      });
    }
  };
  auto read_v = [&](int t, u32x2 (&vh)[KS * DT16 * 2]) __attribute__((always_inline)) {
    const uint32_t bufb = lds0 + (uint32_t)(t % R) * (BUFE * 2);
#pragma unroll
    for (int dt = 0; dt < DT16; ++dt) {
      const uint32_t va = bufb + voff[dt];
      static_for<0, KS>([&](auto ks) __attribute__((always_inline)) {
        constexpr int KSI = decltype(ks)::value;
        vh[(KSI * DT16 + dt) * 2] = ds_read_tr16<KSI * 8192>(va);
        vh[(KSI * DT16 + dt) * 2 + 1] = ds_read_tr16<KSI * 8192 + 4096>(va);
      });
    }
  };
  auto qk = [&](const u32x4 (&kf)[KT * 4], f32x4 (&s)[KT]) __attribute__((always_inline)) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) s[kt] = mfma16<DT>(kf[kt * 4 + ds], qf[ds], s[kt]);
    }
  };
  // the online softmax of block t's scores: P packed for the P.V step; returns whether o must be rescaled
  // by alpha (some query's running maximum moved; alpha = 1 leaves o unchanged bit for bit)
  auto soft = [&](int t, f32x4 (&s)[KT], u32x4 (&pb)[KS], float& alpha) __attribute__((always_inline)) {
    const int k0 = t * KBP + kp0;  // the part's first key from the split's first
    float mx = -INFINITY;
    if (k0 + KPP <= Lks) {
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s[kt][e] *= c2;
          mx = fmaxf(mx, s[kt][e]);
        }
    } else {
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float v = k0 + 16 * kt + 4 * lg + e < Lks ? s[kt][e] * c2 : -INFINITY;
          s[kt][e] = v;
          mx = fmaxf(mx, v);
        }
    }
    mx = rows_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float ps = 0.f;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float pe = __builtin_amdgcn_exp2f(s[kt][e] - m_use);
        s[kt][e] = pe;
        ps += pe;
      }
    ps = rows_sum(ps);
    l_run = l_run * alpha + ps;
    m_run = m_new;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      pb[ks] = u32x4{pack_f32x2<DT>(s[2 * ks][0], s[2 * ks][1]), pack_f32x2<DT>(s[2 * ks][2], s[2 * ks][3]),
                     pack_f32x2<DT>(s[2 * ks + 1][0], s[2 * ks + 1][1]),
                     pack_f32x2<DT>(s[2 * ks + 1][2], s[2 * ks + 1][3])};
  };
  auto pv = [&](const u32x2 (&vh)[KS * DT16 * 2], const u32x4 (&pb)[KS], float alpha) __attribute__((always_inline)) {
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt) o[dt] *= alpha;
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt) {
        const u32x2 h0 = vh[(ks * DT16 + dt) * 2], h1 = vh[(ks * DT16 + dt) * 2 + 1];
        o[dt] = mfma16<DT>(u32x4{h0[0], h0[1], h1[0], h1[1]}, pb[ks], o[dt]);
      }
  };

  // Iteration t: wait for block t + 1's copies (EXACT: every wave issues 2 CPW copies per block, blocks
  // past the last re-read the last, and blocks t + 2 .. t + D - 1 were issued after it), so that its
  // scores can form while block t finishes; the barrier also frees buffer (t - 1) % R (block t - 1's V was
  // read and waited for in iteration t - 1), which takes block t + D.  The scores of block t (cur) were
  // formed in iteration t - 1 (block 0's before the loop).
  f32x4 sa[KT], sb[KT];
  {
    u32x4 kf[KT * 4];
    wait_vmcnt<(D - 1) * 2 * CPW>();  // block 0
    __builtin_amdgcn_s_barrier();
    read_k(0, kf);
    lds_wait(kf);
    qk(kf, sa);
  }
  auto iter = [&](int t, f32x4 (&cur)[KT], f32x4 (&nxt)[KT]) __attribute__((always_inline)) {
    wait_vmcnt<(D - 2) * 2 * CPW>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(t + D);
    u32x4 kf[KT * 4];
    u32x2 vh[KS * DT16 * 2];
    read_k(t + 1, kf);
    read_v(t, vh);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 pb[KS];
    float alpha;
    soft(t, cur, pb, alpha);
    lds_wait(kf);
    lds_wait(vh);
    qk(kf, nxt);
    pv(vh, pb, alpha);
  };
  int t0 = 0;
#pragma nounroll
  for (; t0 + 1 < T; t0 += 2) {
    iter(t0, sa, sb);
    iter(t0 + 1, sb, sa);
  }
  if (t0 < T) iter(t0, sa, sb);
  wait_vmcnt<0>();  // no copy may still be writing LDS when the parts are merged in it

  float L = l_run;
  float Mw = m_run == -INFINITY ? 0.f : m_run;  // o and L are relative to 2^Mw
  if constexpr (KH > 1) {
    // merge the key parts in LDS, in part order (the chunk kernel's merge): parts > 0 leave (m, l) and O^T,
    // part 0 combines them
    __syncthreads();  // every wave is done with the key buffers the merge overwrites
    float* cm = reinterpret_cast<float*>(smem);
    float* cl = cm + KH * NQW * 16;
    f32x4* co = reinterpret_cast<f32x4*>(cl + KH * NQW * 16);
    if (lg == 0) {
      cm[(kh * NQW + qw) * 16 + lr] = m_run;
      cl[(kh * NQW + qw) * 16 + lr] = l_run;
    }
    if (kh > 0) {
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt) co[(((kh - 1) * NQW + qw) * DT16 + dt) * 64 + lane] = o[dt];
    }
    __syncthreads();
    if (kh > 0) return;
    float M = -INFINITY;
    for (int k = 0; k < KH; ++k) M = fmaxf(M, cm[(k * NQW + qw) * 16 + lr]);
    const float Mu = M == -INFINITY ? 0.f : M;
    Mw = Mu;
    L = 0.f;
    for (int k = 0; k < KH; ++k) L += cl[(k * NQW + qw) * 16 + lr] * __builtin_amdgcn_exp2f(cm[(k * NQW + qw) * 16 + lr] - Mu);
    const float f0 = __builtin_amdgcn_exp2f(cm[qw * 16 + lr] - Mu);
#pragma unroll
    for (int dt = 0; dt < DT16; ++dt) o[dt] *= f0;
    for (int k = 1; k < KH; ++k) {
      const float fk = __builtin_amdgcn_exp2f(cm[(k * NQW + qw) * 16 + lr] - Mu);
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt) o[dt] += co[(((k - 1) * NQW + qw) * DT16 + dt) * 64 + lane] * fk;
    }
  }
  if (ns > 1) {
    // key splits: every split's wave leaves (O, m, l) of its query tile by write-through stores; the last to
    // arrive (per sequence, kv head and tile) adds the splits in split order, so which one is last does not
    // change the bits.  The other splits have read their queries from out before they arrived.
    auto slot = [&](int uu) { return p.part + ((size_t)((uu * p.nkv + g) * XG + x) * NQW + qw) * PSZ; };
    float* mine = slot(u0 + js);
#pragma unroll
    for (int dt = 0; dt < DT16; ++dt) stf4<true>(reinterpret_cast<f32x4*>(mine) + dt * 64 + lane, o[dt]);
    if (lg == 0) {
      stf<true>(mine + 16 * HD + lr, Mw);
      stf<true>(mine + 16 * HD + 16 + lr, L);
    }
    wait_memory();  // the stores are acknowledged before the arrival is counted
    unsigned* cnt = p.seq_cnt + ((b * p.nkv + g) * XG + x) * NQW + qw;
    unsigned old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old != (unsigned)(ns - 1)) return;
    if (lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float M = -INFINITY;
    for (int jj = 0; jj < ns; ++jj) M = fmaxf(M, jj == js ? Mw : ldf<true>(slot(u0 + jj) + 16 * HD + lr));
    f32x4 ot[DT16];
#pragma unroll
    for (int dt = 0; dt < DT16; ++dt) ot[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float Lt = 0.f;
    for (int jj = 0; jj < ns; ++jj) {
      const float* q = slot(u0 + jj);
      const float mj = jj == js ? Mw : ldf<true>(q + 16 * HD + lr);
      const float lj = jj == js ? L : ldf<true>(q + 16 * HD + 16 + lr);
      const float f = __builtin_amdgcn_exp2f(mj - M);
      Lt += lj * f;
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt)
        ot[dt] += (jj == js ? o[dt] : ldf4<true>(reinterpret_cast<const f32x4*>(q) + dt * 64 + lane)) * f;
    }
    L = Lt;
#pragma unroll
    for (int dt = 0; dt < DT16; ++dt) o[dt] = ot[dt];
  }
  if (!qvalid) return;
  const float inv = 1.0f / L;
  u16* dst = a.out + (size_t)r * a.nq * HD + (g * grp + hh) * HD + 4 * lg;
#pragma unroll
  for (int dt = 0; dt < DT16; ++dt)
    *reinterpret_cast<u32x2*>(dst + 16 * dt) =
        u32x2{pack_f32x2<DT>(o[dt][0] * inv, o[dt][1] * inv), pack_f32x2<DT>(o[dt][2] * inv, o[dt][3] * inv)};
}

}  // namespace fdllm
