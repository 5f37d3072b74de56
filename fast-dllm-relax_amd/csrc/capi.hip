// C ABI: context, weight binding, workspace, launch planning and the nine entry points.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <initializer_list>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/fdllm.h"
#include "kernels.hpp"
#include "wait_status.hpp"

using namespace fdllm;

namespace {

thread_local std::string g_err;

// Set while fdllm_forward_cached_noalloc runs: a workspace that would have to grow is an error instead
// of an allocation.
thread_local bool t_no_alloc = false;

// The allocation-free cached step's workspace (fdllm_forward_cached_noalloc): one array per GPU, held
// until the process ends.  Host code never uses this name as an address: each device's copy is found
// once with hipGetSymbolAddress (scratch_base) and that pointer is what the kernels receive.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)24 << 20;
constexpr int NOALLOC_MAX_ROWS = 32;
__device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HIPCHK(expr)                                                                  \
  do {                                                                                \
    hipError_t _e = (expr);                                                           \
    if (_e != hipSuccess) return fail(FDLLM_EHIP, "%s: %s", #expr, hipGetErrorString(_e)); \
  } while (0)

struct Layer {
  const uint16_t *wqkv, *bqkv, *wo, *wgu, *wd, *ln_in, *ln_post;  // caller's tensors
  const uint16_t *pqkv, *po, *pgu, *pd;                           // packed copies (context-owned)
};

// A batched call: nseq sequences of `rows` active rows each; sequence b's cache sits seq_stride
// elements after sequence b - 1's in every layer, its rows are written from ws[b] and it attends [0, lk[b]).
struct SeqBatch {
  int nseq; int rows; long long seq_stride;
  int ws[MAX_SEQS]; int lk[MAX_SEQS];
};

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }
int round_up(int x, int a) { return (x + a - 1) / a * a; }

}  // namespace

struct fdllm_ctx {
  fdllm_config cfg;
  int dev = 0;
  std::vector<std::string> names;
  std::vector<const uint16_t*> params;
  bool bound = false;
  std::vector<Layer> layers;
  const uint16_t* embed = nullptr;
  const uint16_t* final_norm = nullptr;
  const uint16_t* lm_head = nullptr;
  uint16_t* packed = nullptr;        // every packed weight matrix, one allocation
  const uint16_t* plm = nullptr;     // packed lm_head
  int lm_tiles = 0;

  // row workspace (grown on demand)
  int ws_rows = 0;
  void* ws = nullptr;
  uint16_t *h = nullptr, *qkv = nullptr, *attn = nullptr, *act = nullptr;
  uint16_t *kscr = nullptr, *vscr = nullptr;  // K/V of a stateless forward (one layer at a time)
  uint16_t* xn = nullptr;                     // RMS-normalised rows for the large-M projections
  float* ssq = nullptr;                       // [hidden / 16][ws_rows] row sums of squares per 16 columns
  // split partials / confidence statistics (grown on demand)
  float* gpart = nullptr; size_t gpart_floats = 0;
  float* apart = nullptr; size_t apart_floats = 0;
  void* stats = nullptr; size_t stats_rows = 0;
  unsigned* counters = nullptr; int n_counters = 0;
  int32_t* zero_i32 = nullptr;
  float* rope = nullptr; size_t rope_floats = 0;  // RoPE (cos, sin) table of the current call's rows
  int attn_target = 64;   // attention workgroups aimed for when splitting the keys
  int prefill_hpw = 0;    // query heads per prefill-attention workgroup (0: chosen per launch)
  int prefill_pair = 1;   // paired-query-block prefill attention (0 off, 1 by size, 2 always all heads, 3 always split)
  int seq_attn = 1;       // batched calls: attn_seq_kernel (0: the chunk kernel with key splits + merge)
  int seq_split = 1;      // attn_seq_kernel splits long sequences' keys over the compute units it leaves idle
  int ncu = 256;          // compute units of the device
  unsigned* attn_cnt = nullptr;  // attn_seq_kernel's arrival counters (SEQ_CNT_MAX, zero between launches)
  int fuse_down = 1;      // large-M down launches with k splits: split sum + residual + next RMSNorm in one launch
  // large-M o_proj with a forced k split and its split sum + residual + the next norm in one launch: -1 with
  // three splits up to 256 rows (128-row batched step: 14.8 + 4.8 us norm -> 8.1 + 7.1 us; at 512 rows it
  // measured slower, 3.88 -> 3.94 ms per step with two splits), 0 never, N > 1 with N splits at any size
  int fuse_oproj = -1;
  // large-M calls whose attention starts with the RoPE / KV-append pass (prefill, batched sequences): that
  // pass done by qkv's epilogue instead (FDLLM_QKV_ROPE=0: the separate pass)
  int qkv_rope = 1;
  int down_split = 10;    // cross-workgroup k splits of the down projection (largest divisor of K/32 <= this)
  MmPolicy mm;              // large-M GEMM planning (k splits, register-weight kernel)
  bool frag_on = true;      // one-shot chains keep activations in MFMA-fragment order (FDLLM_XFRAG=0: row-major)
  // k splits of the one-shot projections summed inside their own launch (GroupWait, kernels.hpp), when the
  // launch's grid is resident at once
  bool group_waits = true;             // FDLLM_GROUP_WAITS=0 turns them off (separate split-sum launches)
  unsigned* gw_cnt = nullptr;          // the counter banks
  unsigned* wait_fault = nullptr;      // host-visible (pinned, mapped) fault word of those waits
  unsigned* wait_fault_dev = nullptr;
  long long wait_limit = 0;            // wall-clock ticks one wait may take (0.2 s)
  long long group_wait_launches = 0;   // launches that reduced their splits themselves (fdllm_group_wait_launches)
  int gw_bank = 0;                     // the bank of the next launch
  int gw_prev = 0;                     // groups the previous launch used (in the other bank)
  long long frag_calls = 0;            // layer loops run in MFMA-fragment order (fdllm_frag_calls)
  unsigned char* scratch_dev = nullptr;  // this device's copy of `scratch` (fdllm_forward_cached_noalloc)

  // the group-wait descriptor of the next launch, which uses `groups` counters
  GroupWait next_group_wait(int groups) {
    GroupWait g{gw_cnt, wait_fault_dev, wait_limit, gw_bank, gw_prev};
    gw_bank ^= 1;
    gw_prev = groups;
    ++group_wait_launches;
    return g;
  }

  int qkv_dim() const { return (cfg.num_attention_heads + 2 * cfg.num_key_value_heads) * cfg.head_dim; }
  int q_dim() const { return cfg.num_attention_heads * cfg.head_dim; }
  int kv_dim() const { return cfg.num_key_value_heads * cfg.head_dim; }
  int tiles() const { return (cfg.vocab_size + 255) / 256; }
  int ssq_tiles() const { return cfg.hidden_size / 16; }
};

namespace {

int ensure_rows(fdllm_ctx* c, int rows) {
  if (rows <= c->ws_rows) return FDLLM_OK;
  if (t_no_alloc)
    return fail(FDLLM_EINVAL, "%d rows exceed the allocation-free step's %d", rows, c->ws_rows);
  int R = (int)align_up((size_t)std::max(rows, 32), 32);
  const fdllm_config& f = c->cfg;
  size_t e_h = (size_t)R * f.hidden_size, e_qkv = (size_t)R * c->qkv_dim(), e_q = (size_t)R * c->q_dim();
  size_t e_act = (size_t)R * f.intermediate_size, e_kv = (size_t)R * c->kv_dim();
  size_t e_ssq = (size_t)c->ssq_tiles() * R * 2;  // floats as u16 pairs
  size_t bytes = 2 * (align_up(e_h, 64) * 2 + align_up(e_qkv, 64) + align_up(e_q, 64) + align_up(e_act, 64) +
                      align_up(e_kv, 64) * 2 + align_up(e_ssq, 64));
  if (c->ws) {
    HIPCHK(hipDeviceSynchronize());
    HIPCHK(hipFree(c->ws));
  }
  c->ws = nullptr;
  HIPCHK(hipMalloc(&c->ws, bytes));
  uint16_t* p = (uint16_t*)c->ws;
  auto take = [&](size_t n) { uint16_t* r = p; p += align_up(n, 64); return r; };
  c->h = take(e_h); c->qkv = take(e_qkv); c->attn = take(e_q); c->act = take(e_act);
  c->kscr = take(e_kv); c->vscr = take(e_kv); c->ssq = (float*)take(e_ssq); c->xn = take(e_h);
  c->ws_rows = R;
  return FDLLM_OK;
}

int ensure_floats(float** buf, size_t* have, size_t need) {
  if (need <= *have) return FDLLM_OK;
  if (t_no_alloc)
    return fail(FDLLM_EINVAL, "the call needs %zu floats of split partials; the allocation-free step's scratch holds %zu",
                need, *have);
  if (*buf) {
    HIPCHK(hipDeviceSynchronize());
    HIPCHK(hipFree(*buf));
  }
  *buf = nullptr;
  size_t n = align_up(need, 1 << 20);
  HIPCHK(hipMalloc((void**)buf, n * sizeof(float)));
  *have = n;
  return FDLLM_OK;
}

int ensure_stats(fdllm_ctx* c, int rows) {
  if ((size_t)rows <= c->stats_rows) return FDLLM_OK;
  size_t R = align_up((size_t)std::max(rows, 32), 32);
  if (c->stats) {
    HIPCHK(hipDeviceSynchronize());
    HIPCHK(hipFree(c->stats));
  }
  c->stats = nullptr;
  HIPCHK(hipMalloc(&c->stats, R * c->tiles() * 12));
  c->stats_rows = R;
  return FDLLM_OK;
}

// Packed tile counts of each projection (padded to whole workgroups of its launch configuration).
int qkv_tiles(const fdllm_ctx* c) { return round_up(c->qkv_dim() / 16, gemm_shape(CFG_QKV).tiles_per_wg); }
int o_tiles(const fdllm_ctx* c) { return round_up(c->cfg.hidden_size / 16, gemm_shape(CFG_OPROJ).tiles_per_wg); }
int gu_tiles(const fdllm_ctx* c) { return round_up(2 * c->cfg.intermediate_size / 16, gemm_shape(CFG_GATE_UP).tiles_per_wg); }
int d_tiles(const fdllm_ctx* c) { return round_up(c->cfg.hidden_size / 16, gemm_shape(CFG_DOWN).tiles_per_wg); }
int lm_tiles_of(const fdllm_ctx* c) { return round_up((c->cfg.vocab_size + 15) / 16, gemm_shape(CFG_LM_HEAD).tiles_per_wg); }

// Largest divisor of n that is <= cap (>= 1).
int divisor_at_most(int n, int cap) {
  for (int d = std::max(1, std::min(n, cap)); d > 1; --d)
    if (n % d == 0) return d;
  return 1;
}

// ksplit: the k split of the streaming kernel (prefill-sized M); the one-shot kernel picks its own.
int run_gemm(fdllm_ctx* c, int cfg, GemmP a, int ksplit, hipStream_t st) {
  const fdllm_config& f = c->cfg;
  if (ksplit < 1 || a.KS % ksplit) return fail(FDLLM_EINVAL, "k split %d does not divide %d k steps", ksplit, a.KS);
  const GemmPlan pl = gemm_plan(cfg, a, ksplit, c->mm);
  if (pl.kind == GK_MM && a.nw != nullptr) {
    // RMSNorm once for all column blocks (the large-M kernel takes normalised rows; the LDS-staged one
    // in its fragment blocks)
    if (a.ldx != a.H || a.KS * 32 != a.H) return fail(FDLLM_EINVAL, "normalised projection input must be [rows, hidden]");
    const int blocks = gemm_takes_blocks(pl) ? 1 : 0;
    HIPCHK(launch_norm_rows(f.dtype, a.X, a.M, a.H, a.ssq, a.ssq_ld, a.nw, a.eps, c->xn, st, 0, blocks));
    a.X = c->xn;
    a.nw = nullptr;
    a.xfrag = blocks ? 2 : 0;
  }
  if (pl.ksplit > 1 || pl.tail_split > 1) {
    int rc = ensure_floats(&c->gpart, &c->gpart_floats, pl.part_floats);
    if (rc) return rc;
    if (pl.groups * pl.mchunks > c->n_counters)
      return fail(FDLLM_EINVAL, "too many GEMM workgroup groups (%d)", pl.groups * pl.mchunks);
    a.part = c->gpart;
    a.counters = c->counters;
    // the one-shot register-fragment body sums its k splits inside the launch when the whole grid is
    // resident at once (one workgroup per compute unit): no split-sum launch
    const long long grid = (long long)pl.groups * pl.ksplit * pl.mchunks;
    if (pl.kind == GK_ONESHOT && cfg != CFG_GATE_UP && gemm_takes_frag(cfg, pl) && pl.tiles_per_wg <= 4 &&
        pl.groups * pl.mchunks <= GW_GROUPS && group_waits_fit(c->group_waits, c->wait_fault, grid, c->ncu)) {
      a.gw = c->next_group_wait(pl.groups * pl.mchunks);
    }
  }
  if (const hipError_t e = launch_gemm(f.dtype, cfg, a, pl, st); e != hipSuccess) {
    // a launch that never ran leaves the counter banks out of step: no more in-launch reductions
    if (a.gw.cnt != nullptr) c->group_waits = false;
    return fail(FDLLM_EHIP, "launch_gemm: %s", hipGetErrorString(e));
  }
  return FDLLM_OK;
}

// An EPI_RESID projection (down, or o_proj) of a large-M call with its k-split sum, residual and the next
// RMSNorm (weight next_w) in one launch after the GEMM (launch_resid_norm) instead of the split-sum launch
// plus a norm_rows launch; y: the normalised rows (yblk: fragment blocks).  Only for launches that split k
// under pol (fused_resid_ok).
int run_resid_fused(fdllm_ctx* c, int cfg, GemmP a, int ksplit, const MmPolicy& pol, const uint16_t* next_w,
                    uint16_t* y, int yblk, hipStream_t st);

GemmP gemm_args(const uint16_t* W, int ntiles, int N, int K, const uint16_t* X, int ldx, int M) {
  GemmP a{};
  a.W = W; a.KS = K / 32; a.ntiles = ntiles; a.N = N; a.X = X; a.ldx = ldx; a.M = M; a.kps = a.KS;
  return a;
}

bool fused_resid_ok(const fdllm_ctx* c, int cfg, GemmP a, int ksplit, const MmPolicy& pol) {
  if (a.nw != nullptr || a.N % 32 || a.N > 2048) return false;
  const GemmPlan pl = gemm_plan(cfg, a, ksplit, pol);
  return pl.kind == GK_MM && pl.ksplit > 1;
}

int run_resid_fused(fdllm_ctx* c, int cfg, GemmP a, int ksplit, const MmPolicy& pol, const uint16_t* next_w,
                    uint16_t* y, int yblk, hipStream_t st) {
  const fdllm_config& f = c->cfg;
  const GemmPlan pl = gemm_plan(cfg, a, ksplit, pol);
  if (pl.kind != GK_MM || pl.ksplit < 2) return fail(FDLLM_EINVAL, "fused residual epilogue needs a k split");
  int rc = ensure_floats(&c->gpart, &c->gpart_floats, std::max(pl.part_floats, (size_t)pl.ksplit * a.M * a.N));
  if (rc) return rc;
  a.part = c->gpart;
  a.counters = c->counters;
  a.part_rows = 1;
  HIPCHK(launch_gemm(f.dtype, cfg, a, pl, st));
  HIPCHK(launch_resid_norm(f.dtype, c->gpart, pl.ksplit, a.M, a.N, (uint16_t*)a.Y, a.ssq_out, a.ssq_ld, next_w,
                           f.rms_norm_eps, y, yblk, st));
  return FDLLM_OK;
}

int run_lm_head(fdllm_ctx* c, const uint16_t* hidden, int rows, float* logits, bool stats, hipStream_t st) {
  const fdllm_config& f = c->cfg;
  GemmP a = gemm_args(c->plm, c->lm_tiles, f.vocab_size, f.hidden_size, hidden, f.hidden_size, rows);
  a.logits = logits; a.ldl = f.vocab_size;
  if (stats) {
    int T = c->tiles();
    char* base = (char*)c->stats;
    a.stat_m = (float*)base;
    a.stat_a = (int32_t*)(base + c->stats_rows * T * 4);
    a.stat_s = (float*)(base + c->stats_rows * T * 8);
    a.stat_tiles = T;
  }
  return run_gemm(c, CFG_LM_HEAD, a, 1, st);
}

// RoPE table of `rows` rows, row r at position pos[r / rows_per_seq] + r % rows_per_seq, shared by every
// layer of the call.
int rope_table(fdllm_ctx* c, int rows, const int32_t* pos, int rows_per_seq, hipStream_t st) {
  int rc = ensure_floats(&c->rope, &c->rope_floats, (size_t)rows * 128);
  if (rc) return rc;
  HIPCHK(launch_rope_table(c->cfg.dtype, pos, rows, rows_per_seq, (float)(-std::log((double)c->cfg.rope_theta)),
                           c->rope, st));
  return FDLLM_OK;
}

// The attention launch of the call's rows, planned into a; the RoPE table (rope_table) must hold the
// call's positions.  With sb, the rows are sb->nseq sequences of sb->rows (ws and Lk are then ignored).
int plan_attention(fdllm_ctx* c, AttnP& a, int rows, uint16_t* kc, uint16_t* vc, int ws, int Lk, int mask,
                   const float* bias, long long bias_ld, const SeqBatch* sb, bool frag) {
  const fdllm_config& f = c->cfg;
  a = AttnP{};
  a.qkv = c->qkv; a.ldq = c->qkv_dim(); a.rows = rows; a.nq = f.num_attention_heads; a.nkv = f.num_key_value_heads;
  a.rope = c->rope;
  a.kc = kc; a.vc = vc; a.ws = ws; a.Lk = Lk; a.scale = 1.0f / std::sqrt((float)f.head_dim);
  a.mask = mask; a.q_pos0 = 0; a.block = f.bd_size; a.bias = bias; a.bias_ld = bias_ld;
  a.nseq = 1;
  int target = c->attn_target;
  if (sb != nullptr) {
    a.nseq = sb->nseq; a.rows = sb->rows; a.seq_stride = sb->seq_stride;
    a.ws = 0; a.Lk = 0;
    for (int b = 0; b < sb->nseq; ++b) {
      a.seq_ws[b] = sb->ws[b]; a.seq_lk[b] = sb->lk[b];
      a.ws = std::max(a.ws, sb->ws[b]); a.Lk = std::max(a.Lk, sb->lk[b]);
    }
    target = std::max(1, target / sb->nseq);
  }
  const AttnPlan pl = attn_plan(a.rows, a.nq, a.nkv, a.Lk, target, a.nseq);
  // batched calls without a mask take attn_seq_kernel (every key of a sequence in one workgroup, no
  // partials) from 32 rows per sequence, or when the chunk plan cannot cover the longest sequence in one
  // step; otherwise the chunk kernel.  Measured on config 4 (16 sequences, prefixes up to 1024): 32 rows
  // 17.0 + 4.8 us (RoPE / KV append pass) against 22.2 + 8.4 us (chunks + merge); at 8 rows the chunk
  // kernel keeps the job (11.4 + 4.3 us: each workgroup of this kernel walks all of its sequence's keys)
  const bool seq_kernel = sb != nullptr && c->seq_attn && mask == 0 && (sb->rows >= 32 || !pl.chunked);
  if (sb != nullptr && !seq_kernel && !pl.chunked)
    return fail(FDLLM_EINVAL, "batched call of %d rows per sequence over %d keys is too long for one step", a.rows, a.Lk);
  a.S = pl.S; a.chunk = pl.chunk; a.target_wgs = target; a.prefill_hpw = c->prefill_hpw; a.prefill_pair = c->prefill_pair;
  a.seq_attn = seq_kernel;
  if (seq_kernel) {
    a.seq_cnt = c->attn_cnt;
    const size_t pf = plan_seq_units(a, c->seq_split ? c->ncu : 0);
    if (pf) {
      int rc = ensure_floats(&c->apart, &c->apart_floats, pf);
      if (rc) return rc;
      a.part = c->apart;
    }
  }
  if (a.S > 1 && !seq_kernel) {
    int rc = ensure_floats(&c->apart, &c->apart_floats, attn_partial_floats(a));
    if (rc) return rc;
    a.part = c->apart;
  }
  a.out = c->attn;
  a.ofrag = frag;
  return FDLLM_OK;
}

int run_attention(fdllm_ctx* c, int rows, uint16_t* kc, uint16_t* vc, int ws, int Lk, int mask,
                  const float* bias, long long bias_ld, hipStream_t st, const SeqBatch* sb = nullptr, bool frag = false) {
  AttnP a;
  int rc = plan_attention(c, a, rows, kc, vc, ws, Lk, mask, bias, bias_ld, sb, frag);
  if (rc) return rc;
  HIPCHK(launch_attention(c->cfg.dtype, a, st));
  return FDLLM_OK;
}

// The four projections of layer L at `rows` rows, as the layer loop launches them.  frag: the one-shot
// chain's activations (h, the attention output, SiLU * up) are in MFMA-fragment order.
struct LayerGemms { GemmP q, o, gu, d; int dsplit; };
LayerGemms layer_gemms(const fdllm_ctx* c, const Layer& L, int rows, bool frag) {
  const fdllm_config& f = c->cfg;
  const int H = f.hidden_size, I = f.intermediate_size, ssq_ld = c->ws_rows;
  LayerGemms g;
  g.q = gemm_args(L.pqkv, qkv_tiles(c), c->qkv_dim(), H, c->h, H, rows);
  g.q.ssq = c->ssq; g.q.ssq_tiles = c->ssq_tiles(); g.q.ssq_ld = ssq_ld; g.q.nw = L.ln_in; g.q.eps = f.rms_norm_eps;
  g.q.H = H; g.q.Y = c->qkv; g.q.ldy = c->qkv_dim(); g.q.bias = L.bqkv;
  g.q.xfrag = frag;
  g.o = gemm_args(L.po, o_tiles(c), H, c->q_dim(), c->attn, c->q_dim(), rows);
  g.o.Y = c->h; g.o.ldy = H; g.o.ssq_out = c->ssq; g.o.ssq_ld = ssq_ld;
  g.o.xfrag = g.o.yfrag = frag;
  g.gu = gemm_args(L.pgu, gu_tiles(c), I, H, c->h, H, rows);
  g.gu.ssq = c->ssq; g.gu.ssq_tiles = c->ssq_tiles(); g.gu.ssq_ld = ssq_ld; g.gu.nw = L.ln_post;
  g.gu.eps = f.rms_norm_eps; g.gu.H = H; g.gu.Y = c->act; g.gu.ldy = I;
  g.gu.xfrag = g.gu.yfrag = frag;
  g.d = gemm_args(L.pd, d_tiles(c), H, I, c->act, I, rows);
  g.d.Y = c->h; g.d.ldy = H; g.d.ssq_out = c->ssq; g.d.ssq_ld = ssq_ld;
  g.d.xfrag = g.d.yfrag = frag;
  g.dsplit = divisor_at_most(I / 32, c->down_split);
  if (!frag && rows > 32) {
    // large M: when gate_up and down both run the LDS-staged kernel, SiLU * up goes straight into the
    // fragment blocks down copies
    GemmP tg = g.gu, td = g.d;
    const GemmPlan pg = gemm_plan(CFG_GATE_UP, tg, 1, c->mm);
    const GemmPlan pd = gemm_plan(CFG_DOWN, td, g.dsplit, c->mm);
    if (gemm_takes_blocks(pg) && gemm_takes_blocks(pd)) g.gu.yfrag = g.d.xfrag = 2;
  }
  return g;
}

// Whether a call of `rows` rows runs every projection in the one-shot register-fragment body, so that its
// activations can stay in MFMA-fragment order from load_rows to the final norm.
bool frag_chain(const fdllm_ctx* c, int rows) {
  if (!c->frag_on || rows > 32) return false;
  LayerGemms g = layer_gemms(c, c->layers[0], rows, false);
  const std::pair<int, GemmP*> all[] = {{CFG_QKV, &g.q}, {CFG_OPROJ, &g.o}, {CFG_GATE_UP, &g.gu}, {CFG_DOWN, &g.d}};
  for (const auto& [cfg, a] : all) {
    GemmP t = *a;
    const GemmPlan pl = gemm_plan(cfg, t, cfg == CFG_DOWN ? g.dsplit : 1, c->mm);
    if (!gemm_takes_frag(cfg, pl)) return false;
  }
  return true;
}

// The decoder-layer loop (cuda.py:561-579 per layer, 639-666 for the model).
//   per layer: qkv (RMSNorm on load, + bias) -> attention (RoPE, KV append, GQA) -> o_proj + residual
//              -> gate_up (RMSNorm on load, SiLU * up) -> down + residual
// kv: per-layer cache base pointers are k/v + layer * layer_stride (elements).  out == nullptr skips
// the final norm (build_prefix_cache returns only the caches).
// sb: a batched call (rows = sb->nseq x sb->rows; pos_dev holds one offset per sequence).
int run_layers(fdllm_ctx* c, const void* x_in, int rows, uint16_t* kbase, uint16_t* vbase, size_t layer_stride,
               int write_start, const int32_t* pos_dev, int attend_len, int mask, const float* bias,
               long long bias_ld, void* out, hipStream_t st, const SeqBatch* sb = nullptr) {
  const fdllm_config& f = c->cfg;
  const int H = f.hidden_size;
  const int ssq_ld = c->ws_rows;
  // batched calls keep the activations row-major
  const bool frag = sb == nullptr && frag_chain(c, rows);
  HIPCHK(launch_load_rows(f.dtype, (const uint16_t*)x_in, rows, H, c->h, c->ssq, ssq_ld, st, frag));
  int rc = rope_table(c, rows, pos_dev, sb ? sb->rows : rows, st);
  if (rc) return rc;
  if (frag) ++c->frag_calls;
  // xn_ready: the previous layer's down launch also normalised this layer's qkv input into c->xn
  // (run_resid_fused), in the layout the qkv launch takes; final_done: the last one wrote out
  bool xn_ready = false, final_done = false;
  int xn_layout = 0;
  for (int l = 0; l < f.num_hidden_layers; ++l) {
    const Layer& L = c->layers[l];
    uint16_t* kc = kbase + (size_t)l * layer_stride;
    uint16_t* vc = vbase + (size_t)l * layer_stride;
    LayerGemms g = layer_gemms(c, L, rows, frag);
    if (xn_ready) {
      g.q.X = c->xn;
      g.q.nw = nullptr;
      g.q.xfrag = xn_layout;
    }
    AttnP at;
    rc = plan_attention(c, at, rows, kc, vc, write_start, attend_len, mask, bias, bias_ld, sb, frag);
    if (rc) return rc;
    if (!frag && rows > 32 && c->qkv_rope && attn_takes_roped(at)) {
      // the queries RoPE'd and the K/V rows appended by qkv's epilogue, when its kernel takes that
      GemmP tq = g.q;
      const GemmPlan pq = gemm_plan(CFG_QKV, tq, 1, c->mm);
      if (gemm_ropes_in_epilogue(CFG_QKV, pq) && g.q.ntiles % 8 == 0) {
        RopeOut& ro = g.q.ro;
        ro.rope = c->rope; ro.q = at.out; ro.kc = kc; ro.vc = vc;
        ro.nq = f.num_attention_heads; ro.nkv = f.num_key_value_heads;
        ro.rows = at.nseq > 1 ? at.rows : rows;
        ro.seq_stride = at.nseq > 1 ? at.seq_stride : 0;
        for (int b = 0; b < at.nseq; ++b) ro.ws[b] = at.nseq > 1 ? at.seq_ws[b] : at.ws;
        at.roped = 1;
      }
    }
    rc = run_gemm(c, CFG_QKV, g.q, 1, st);
    if (rc) return rc;
    HIPCHK(launch_attention(f.dtype, at, st));
    // o_proj + the post-attention norm: with a forced k split, when gate_up takes normalised rows
    bool gu_ready = false;
    const int oproj_split = c->fuse_oproj > 1 ? c->fuse_oproj : (c->fuse_oproj < 0 && rows <= 256 ? 3 : 0);
    if (!frag && oproj_split > 1) {
      MmPolicy po = c->mm;
      po.force_split = oproj_split;
      GemmP tg = g.gu;
      const GemmPlan pg = gemm_plan(CFG_GATE_UP, tg, 1, c->mm);
      if (pg.kind == GK_MM && fused_resid_ok(c, CFG_OPROJ, g.o, 1, po)) {
        const int lay = gemm_takes_blocks(pg) ? 2 : 0;
        rc = run_resid_fused(c, CFG_OPROJ, g.o, 1, po, L.ln_post, c->xn, lay, st);
        if (rc) return rc;
        g.gu.X = c->xn;
        g.gu.nw = nullptr;
        g.gu.xfrag = lay;
        gu_ready = true;
      }
    }
    if (!gu_ready) {
      rc = run_gemm(c, CFG_OPROJ, g.o, 1, st);
      if (rc) return rc;
    }
    rc = run_gemm(c, CFG_GATE_UP, g.gu, 1, st);
    if (rc) return rc;
    xn_ready = false;
    if (!frag && c->fuse_down && fused_resid_ok(c, CFG_DOWN, g.d, g.dsplit, c->mm)) {
      if (l + 1 < f.num_hidden_layers) {
        // the next layer's qkv: its launch takes normalised rows (row-major or fragment blocks)
        GemmP tq = layer_gemms(c, c->layers[l + 1], rows, frag).q;
        const GemmPlan pq = gemm_plan(CFG_QKV, tq, 1, c->mm);
        if (pq.kind == GK_MM) {
          xn_layout = gemm_takes_blocks(pq) ? 2 : 0;
          rc = run_resid_fused(c, CFG_DOWN, g.d, g.dsplit, c->mm, c->layers[l + 1].ln_in, c->xn, xn_layout, st);
          if (rc) return rc;
          xn_ready = true;
          continue;
        }
      } else if (out != nullptr) {
        rc = run_resid_fused(c, CFG_DOWN, g.d, g.dsplit, c->mm, c->final_norm, (uint16_t*)out, 0, st);
        if (rc) return rc;
        final_done = true;
        continue;
      }
    }
    rc = run_gemm(c, CFG_DOWN, g.d, g.dsplit, st);
    if (rc) return rc;
  }
  if (out != nullptr && !final_done)
    HIPCHK(launch_norm_rows(f.dtype, c->h, rows, H, c->ssq, ssq_ld, c->final_norm, f.rms_norm_eps, (uint16_t*)out, st, frag));
  return FDLLM_OK;
}

// Activations, caches and logits are read and written in 16-byte units (the caches also by 16-byte
// global-to-LDS copies): such a tensor argument that is not 16-byte aligned is refused.
int check_aligned(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (p != nullptr && (uintptr_t)p % 16)
      return fail(FDLLM_EINVAL, "tensor arguments (activations, caches, logits) must be 16-byte aligned");
  return FDLLM_OK;
}

int check_ready(const fdllm_ctx* c) {
  if (!c) return fail(FDLLM_EINVAL, "null context");
  if (!c->bound) return fail(FDLLM_ESTATE, "weights are not bound (fdllm_bind_weights)");
  return FDLLM_OK;
}

// A group wait of an earlier launch timed out (its outputs are wrong): report it once and reduce every
// split with the separate kernels from now on (wait_status.hpp).
int pending_wait_fault(fdllm_ctx* c) {
  if (take_wait_fault(c->wait_fault, &c->group_waits))
    return fail(FDLLM_EHIP, "a group wait of an earlier launch timed out; the results of that call are invalid");
  return FDLLM_OK;
}

int cached_step(fdllm_ctx* c, const void* x, int rows, void* k, void* v, int cap, const int32_t* off,
                int64_t prefix_len, int write_rel, int attend_rel, void* out, void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  rc = pending_wait_fault(c);
  if (rc) return rc;
  if (!x || !k || !v || !off || !out) return fail(FDLLM_EINVAL, "null tensor argument");
  rc = check_aligned({x, k, v, out});
  if (rc) return rc;
  if (rows <= 0) return fail(FDLLM_EINVAL, "active rows must be positive, got %d", rows);
  int64_t write_start = prefix_len + write_rel, attend_len = prefix_len + attend_rel;
  // fast_dllm.attn_inplace guard (runtime.py:69-70) and the write-window check (runtime.py:56-57)
  if (write_start + rows > attend_len)
    return fail(FDLLM_EINVAL, "KV write [%lld, %lld) past the attended rows [0, %lld)", (long long)write_start,
                (long long)(write_start + rows), (long long)attend_len);
  if (write_start < 0 || write_start + rows > cap)
    return fail(FDLLM_EINVAL, "KV write [%lld, %lld) outside cache capacity %d", (long long)write_start,
                (long long)(write_start + rows), cap);
  // the attended rows must exist too (_check_write, runtime.py:262-263)
  if (attend_len > cap)
    return fail(FDLLM_EINVAL, "cached call needs %lld rows; cache capacity is %d", (long long)attend_len, cap);
  rc = ensure_rows(c, rows);
  if (rc) return rc;
  const fdllm_config& f = c->cfg;
  size_t stride = (size_t)cap * f.num_key_value_heads * f.head_dim;
  return run_layers(c, x, rows, (uint16_t*)k, (uint16_t*)v, stride, (int)write_start, off, (int)attend_len, 0,
                    nullptr, 0, out, (hipStream_t)stream);
}

// Batched cached step over nseq sequences sharing one cache tensor [L, nseq, cap, nkv, hd]: the checks
// of cached_step per sequence, then one pass of the layers over nseq x rows rows.
int cached_step_batch(fdllm_ctx* c, const void* x, int nseq, int rows, void* k, void* v, int cap, const int32_t* off,
                      const int64_t* prefix_lens, int write_rel, int attend_rel, void* out, void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  rc = pending_wait_fault(c);
  if (rc) return rc;
  if (!x || !k || !v || !off || !prefix_lens || !out) return fail(FDLLM_EINVAL, "null tensor argument");
  rc = check_aligned({x, k, v, out});
  if (rc) return rc;
  if (nseq <= 0 || nseq > MAX_SEQS) return fail(FDLLM_EINVAL, "batch of %d sequences (1 .. %d supported)", nseq, MAX_SEQS);
  if (rows <= 0) return fail(FDLLM_EINVAL, "active rows must be positive, got %d", rows);
  const fdllm_config& f = c->cfg;
  SeqBatch sb{};
  sb.nseq = nseq; sb.rows = rows; sb.seq_stride = (long long)cap * f.num_key_value_heads * f.head_dim;
  for (int b = 0; b < nseq; ++b) {
    const int64_t ws = prefix_lens[b] + write_rel, lk = prefix_lens[b] + attend_rel;
    if (ws + rows > lk)
      return fail(FDLLM_EINVAL, "sequence %d: KV write [%lld, %lld) past the attended rows [0, %lld)", b, (long long)ws,
                  (long long)(ws + rows), (long long)lk);
    if (ws < 0 || ws + rows > cap)
      return fail(FDLLM_EINVAL, "sequence %d: KV write [%lld, %lld) outside cache capacity %d", b, (long long)ws,
                  (long long)(ws + rows), cap);
    if (lk > cap) return fail(FDLLM_EINVAL, "sequence %d: cached call needs %lld rows; cache capacity is %d", b,
                              (long long)lk, cap);
    sb.ws[b] = (int)ws;
    sb.lk[b] = (int)lk;
  }
  rc = ensure_rows(c, nseq * rows);
  if (rc) return rc;
  const size_t layer_stride = (size_t)nseq * sb.seq_stride;
  return run_layers(c, x, nseq * rows, (uint16_t*)k, (uint16_t*)v, layer_stride, 0, off, 0, 0, nullptr, 0, out,
                    (hipStream_t)stream, &sb);
}

int pack_all(fdllm_ctx* c) {
  const fdllm_config& f = c->cfg;
  const int H = f.hidden_size, I = f.intermediate_size;
  const size_t per_layer = (size_t)qkv_tiles(c) * (H / 32) * 512 + (size_t)o_tiles(c) * (c->q_dim() / 32) * 512 +
                           (size_t)gu_tiles(c) * (H / 32) * 512 + (size_t)d_tiles(c) * (I / 32) * 512;
  c->lm_tiles = lm_tiles_of(c);
  const size_t lm = (size_t)c->lm_tiles * (H / 32) * 512;
  if (c->packed == nullptr) HIPCHK(hipMalloc((void**)&c->packed, (per_layer * f.num_hidden_layers + lm) * 2));
  uint16_t* p = c->packed;
  for (int l = 0; l < f.num_hidden_layers; ++l) {
    Layer& L = c->layers[l];
    HIPCHK(launch_pack(L.wqkv, c->qkv_dim(), H, qkv_tiles(c), PACK_ROWS, p, nullptr));
    L.pqkv = p; p += (size_t)qkv_tiles(c) * (H / 32) * 512;
    HIPCHK(launch_pack(L.wo, H, c->q_dim(), o_tiles(c), PACK_ROWS, p, nullptr));
    L.po = p; p += (size_t)o_tiles(c) * (c->q_dim() / 32) * 512;
    HIPCHK(launch_pack(L.wgu, 2 * I, H, gu_tiles(c), PACK_PAIRS, p, nullptr));
    L.pgu = p; p += (size_t)gu_tiles(c) * (H / 32) * 512;
    HIPCHK(launch_pack(L.wd, H, I, d_tiles(c), PACK_ROWS, p, nullptr));
    L.pd = p; p += (size_t)d_tiles(c) * (I / 32) * 512;
  }
  HIPCHK(launch_pack(c->lm_head, f.vocab_size, H, c->lm_tiles, PACK_ROWS, p, nullptr));
  c->plm = p;
  HIPCHK(hipDeviceSynchronize());
  return FDLLM_OK;
}

}  // namespace

extern "C" {

const char* fdllm_last_error(void) { return g_err.c_str(); }

int fdllm_create(const fdllm_config* cfg, fdllm_ctx** out) {
  if (!cfg || !out) return fail(FDLLM_EINVAL, "null argument");
  const fdllm_config& f = *cfg;
  if (f.dtype != FDLLM_DTYPE_BF16 && f.dtype != FDLLM_DTYPE_F16) return fail(FDLLM_EINVAL, "unsupported dtype %d", f.dtype);
  if (f.head_dim != 128) return fail(FDLLM_EINVAL, "head_dim %d unsupported (the attention kernel is built for 128)", f.head_dim);
  if (f.num_attention_heads <= 0 || f.num_key_value_heads <= 0 || f.num_attention_heads % f.num_key_value_heads)
    return fail(FDLLM_EINVAL, "num_attention_heads must be a positive multiple of num_key_value_heads");
  if (f.hidden_size % 128 || f.intermediate_size % 128 || (f.num_attention_heads * f.head_dim) % 128)
    return fail(FDLLM_EINVAL, "hidden_size, intermediate_size and q width must be multiples of 128");
  if (f.hidden_size > 2048) return fail(FDLLM_EINVAL, "hidden_size %d above the lm_head kernel's 2048", f.hidden_size);
  if (f.vocab_size <= 0 || f.num_hidden_layers <= 0 || f.bd_size <= 0 || f.bd_size % 4)
    return fail(FDLLM_EINVAL, "invalid vocab/layers/bd_size");
  fdllm_ctx* c = new fdllm_ctx();
  c->cfg = f;
  (void)hipGetDevice(&c->dev);
  if (const char* e = std::getenv("FDLLM_ATTN_TARGET")) c->attn_target = std::max(1, atoi(e));
  if (const char* e = std::getenv("FDLLM_PREFILL_HPW")) c->prefill_hpw = std::max(0, atoi(e));
  if (const char* e = std::getenv("FDLLM_PREFILL_PAIR")) c->prefill_pair = std::min(3, std::max(0, atoi(e)));
  if (const char* e = std::getenv("FDLLM_SEQ_ATTN")) c->seq_attn = atoi(e) != 0;
  if (const char* e = std::getenv("FDLLM_FUSE_DOWN")) c->fuse_down = atoi(e) != 0;
  if (const char* e = std::getenv("FDLLM_FUSE_OPROJ")) c->fuse_oproj = e[0] != '\0' ? std::max(0, atoi(e)) : -1;
  if (const char* e = std::getenv("FDLLM_QKV_ROPE")) c->qkv_rope = atoi(e) != 0;
  if (const char* e = std::getenv("FDLLM_DOWN_SPLIT")) c->down_split = std::max(1, atoi(e));
  if (const char* e = std::getenv("FDLLM_MM_TARGET_WGS")) c->mm.target_wgs = std::max(1, atoi(e));
  if (const char* e = std::getenv("FDLLM_MM_MIN_STAGES")) c->mm.min_stages = std::max(1, atoi(e));
  if (const char* e = std::getenv("FDLLM_WR_OPS")) c->mm.wr_ops = atoi(e) & 31;
  if (const char* e = std::getenv("FDLLM_WR_MIN_ROWS")) c->mm.wr_min_rows = std::max(0, atoi(e));
  if (const char* e = std::getenv("FDLLM_WR_SMALL")) c->mm.wr_small_ops = atoi(e) & 3;
  if (const char* e = std::getenv("FDLLM_WR_FFN")) c->mm.wr_ffn = e[0] != '\0' ? (atoi(e) & 15) : -1;
  if (const char* e = std::getenv("FDLLM_WR3")) c->mm.wr3 = atoi(e) != 0;
  if (const char* e = std::getenv("FDLLM_SEQ_SPLIT")) c->seq_split = atoi(e) != 0;
  if (const char* e = std::getenv("FDLLM_WT8")) c->mm.wt8 = atoi(e);
  if (const char* e = std::getenv("FDLLM_WT256")) c->mm.wt256 = atoi(e);
  if (const char* e = std::getenv("FDLLM_GROUP_WAITS")) c->group_waits = atoi(e) != 0;
  if (const char* e = std::getenv("FDLLM_XFRAG")) c->frag_on = atoi(e) != 0;
  if (const char* e = std::getenv("FDLLM_OS_HALF")) c->mm.os_half = atoi(e) & 3;
  // fp16 keeps whole 32-row chunks: its norm transform compiles to a different mix of fp16 rounding
  // instructions (v_fma_mixlo_f16 or an fp32 multiply and a conversion) for 16-row chunks, which changed
  // results in the last bit; no fp16 workload here runs the one-shot chain at 17-32 rows
  if (f.dtype == FDLLM_DTYPE_F16) c->mm.os_half = 0;
  c->names.push_back("model.embed_tokens.weight");
  for (int i = 0; i < f.num_hidden_layers; ++i) {
    std::string p = "model.layers." + std::to_string(i);
    for (const char* s : {".self_attn.qkv_proj.weight", ".self_attn.qkv_proj.bias", ".self_attn.o_proj.weight",
                          ".mlp.gate_up_proj.weight", ".mlp.down_proj.weight", ".input_layernorm.weight",
                          ".post_attention_layernorm.weight"})
      c->names.push_back(p + s);
  }
  c->names.push_back("model.norm.weight");
  if (!f.tie_word_embeddings) c->names.push_back("lm_head.weight");
  c->n_counters = 1 << 16;
  constexpr size_t gw_words = (size_t)2 * GW_GROUPS * GW_STRIDE;  // two banks of group counters
  const size_t cnt_bytes = ((size_t)c->n_counters + SEQ_CNT_MAX + gw_words) * 4 + 64;
  hipError_t e = hipMalloc((void**)&c->counters, cnt_bytes);
  if (e == hipSuccess) e = hipMemset(c->counters, 0, cnt_bytes);
  if (e != hipSuccess) {
    delete c;
    return fail(FDLLM_EHIP, "workspace allocation failed: %s", hipGetErrorString(e));
  }
  c->attn_cnt = c->counters + c->n_counters;
  c->gw_cnt = c->attn_cnt + SEQ_CNT_MAX;
  c->zero_i32 = (int32_t*)(c->gw_cnt + gw_words);
  {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, c->dev) == hipSuccess && cus > 0) c->ncu = cus;
    else (void)hipGetLastError();
    c->mm.lm_tail_cus = c->ncu;
    if (const char* e = std::getenv("FDLLM_LM_TAIL")) c->mm.lm_tail_cus = atoi(e) != 0 ? c->ncu : 0;
  }
  {
    // this device's copy of the allocation-free step's scratch array, found once per device
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (c->dev >= 0 && c->dev < MAX_DEVICES) {
      if (g_scratch_ptr[c->dev] == nullptr) {
        void* ptr = nullptr;
        const hipError_t se = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (se != hipSuccess) {
          (void)hipGetLastError();
          ptr = nullptr;  // the allocation-free entry point then reports that it is unavailable
        }
        g_scratch_ptr[c->dev] = ptr;
      }
      c->scratch_dev = (unsigned char*)g_scratch_ptr[c->dev];
    }
  }
  {
    // the fault word of the group waits; without it every split is reduced by a separate kernel
    int khz = 0;
    (void)hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, c->dev);
    c->wait_limit = (long long)std::max(khz, 1000) * 200;  // 0.2 s
    if (hipHostMalloc((void**)&c->wait_fault, 64, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
        hipHostGetDevicePointer((void**)&c->wait_fault_dev, c->wait_fault, 0) != hipSuccess) {
      (void)hipGetLastError();
      if (c->wait_fault) (void)hipHostFree(c->wait_fault);
      c->wait_fault = c->wait_fault_dev = nullptr;
      c->group_waits = false;
    } else {
      *c->wait_fault = 0u;
    }
  }
  int rc = ensure_rows(c, std::max(1, f.max_rows));
  if (rc == FDLLM_OK) rc = ensure_stats(c, std::max(32, f.max_rows));
  if (rc == FDLLM_OK) {
    e = hipDeviceSynchronize();
    if (e != hipSuccess) rc = fail(FDLLM_EHIP, "%s", hipGetErrorString(e));
  }
  if (rc) {
    fdllm_destroy(c);
    return rc;
  }
  *out = c;
  return FDLLM_OK;
}

void fdllm_destroy(fdllm_ctx* c) {
  if (!c) return;
  (void)hipDeviceSynchronize();
  for (void* p : {c->ws, (void*)c->gpart, (void*)c->apart, c->stats, (void*)c->counters, (void*)c->packed,
                  (void*)c->rope})
    if (p) (void)hipFree(p);
  if (c->wait_fault) (void)hipHostFree(c->wait_fault);
  delete c;
}

int fdllm_num_params(const fdllm_ctx* c) { return c ? (int)c->names.size() : 0; }

const char* fdllm_param_name(const fdllm_ctx* c, int i) {
  if (!c || i < 0 || i >= (int)c->names.size()) return nullptr;
  return c->names[i].c_str();
}

int fdllm_bind_weights(fdllm_ctx* c, const void* const* ptrs, int n) {
  if (!c || !ptrs) return fail(FDLLM_EINVAL, "null argument");
  if (n != (int)c->names.size()) return fail(FDLLM_EINVAL, "expected %d params, got %d", (int)c->names.size(), n);
  for (int i = 0; i < n; ++i) {
    if (!ptrs[i]) return fail(FDLLM_EINVAL, "param %d (%s) is null", i, c->names[i].c_str());
    // the kernels read norm weights, biases and embedding rows with 16-byte loads
    if ((uintptr_t)ptrs[i] % 16)
      return fail(FDLLM_EINVAL, "param %d (%s) is not 16-byte aligned", i, c->names[i].c_str());
  }
  c->params.assign((const uint16_t* const*)ptrs, (const uint16_t* const*)ptrs + n);
  c->embed = c->params[0];
  c->layers.resize(c->cfg.num_hidden_layers);
  for (int i = 0; i < c->cfg.num_hidden_layers; ++i) {
    const uint16_t* const* p = &c->params[1 + 7 * i];
    c->layers[i] = Layer{p[0], p[1], p[2], p[3], p[4], p[5], p[6], nullptr, nullptr, nullptr, nullptr};
  }
  c->final_norm = c->params[1 + 7 * c->cfg.num_hidden_layers];
  c->lm_head = c->cfg.tie_word_embeddings ? c->embed : c->params[2 + 7 * c->cfg.num_hidden_layers];
  c->bound = false;
  int rc = pack_all(c);
  if (rc) return rc;
  c->bound = true;
  return FDLLM_OK;
}

int fdllm_embed(fdllm_ctx* c, const int32_t* ids, int n, void* out, void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  if (n <= 0) return fail(FDLLM_EINVAL, "seq_len must be positive, got %d", n);
  if (!ids || !out) return fail(FDLLM_EINVAL, "null tensor argument");
  HIPCHK(launch_embed(ids, n, c->embed, c->cfg.vocab_size, c->cfg.hidden_size, (uint16_t*)out, (hipStream_t)stream));
  return FDLLM_OK;
}

int fdllm_forward_hidden(fdllm_ctx* c, const void* x, int S, const float* bias, void* out, void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  rc = pending_wait_fault(c);
  if (rc) return rc;
  if (S <= 0) return fail(FDLLM_EINVAL, "seq_len must be positive, got %d", S);
  if (!x || !out) return fail(FDLLM_EINVAL, "null tensor argument");
  rc = check_aligned({x, out});
  if (rc) return rc;
  rc = ensure_rows(c, S);
  if (rc) return rc;
  return run_layers(c, x, S, c->kscr, c->vscr, 0, 0, c->zero_i32, S, bias ? 2 : 1, bias, S, out, (hipStream_t)stream);
}

int fdllm_get_logits(fdllm_ctx* c, const void* hidden, int rows, float* logits, void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  rc = pending_wait_fault(c);
  if (rc) return rc;
  if (rows <= 0 || !hidden || !logits) return fail(FDLLM_EINVAL, "invalid get_logits arguments");
  rc = check_aligned({hidden, logits});
  if (rc) return rc;
  return run_lm_head(c, (const uint16_t*)hidden, rows, logits, false, (hipStream_t)stream);
}

int fdllm_build_prefix_cache(fdllm_ctx* c, const void* x, int P, const float* bias, void* k, void* v, int cap,
                             void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  rc = pending_wait_fault(c);
  if (rc) return rc;
  if (P <= 0 || !x || !k || !v) return fail(FDLLM_EINVAL, "invalid build_prefix_cache arguments");
  rc = check_aligned({x, k, v});
  if (rc) return rc;
  if (P > cap) return fail(FDLLM_EINVAL, "KV write [0, %d) outside cache capacity %d", P, cap);
  rc = ensure_rows(c, P);
  if (rc) return rc;
  const fdllm_config& f = c->cfg;
  size_t stride = (size_t)cap * f.num_key_value_heads * f.head_dim;
  // build_prefix_cache returns only the caches: no final norm
  return run_layers(c, x, P, (uint16_t*)k, (uint16_t*)v, stride, 0, c->zero_i32, P, bias ? 2 : 1, bias, P, nullptr,
                    (hipStream_t)stream);
}

int fdllm_forward_cached(fdllm_ctx* c, const void* x, int rows, void* k, void* v, int cap, const int32_t* off,
                         int64_t prefix_len, void* out, void* stream) {
  return cached_step(c, x, rows, k, v, cap, off, prefix_len, 0, rows, out, stream);
}

// The workspace a call of the allocation-free step sees: views of this device's scratch array swapped
// into the context for the duration of the call (the context is single-threaded by contract) and
// restored after it, with t_no_alloc turning any growth into an error.
struct ScratchView {
  fdllm_ctx* c;
  uint16_t *h, *qkv, *attn, *act, *kscr, *vscr, *xn;
  float *ssq, *gpart, *apart, *rope;
  size_t gpart_floats, apart_floats, rope_floats;
  int ws_rows;
  explicit ScratchView(fdllm_ctx* ctx) : c(ctx) {
    h = c->h; qkv = c->qkv; attn = c->attn; act = c->act; kscr = c->kscr; vscr = c->vscr; xn = c->xn;
    ssq = c->ssq; gpart = c->gpart; apart = c->apart; rope = c->rope;
    gpart_floats = c->gpart_floats; apart_floats = c->apart_floats; rope_floats = c->rope_floats;
    ws_rows = c->ws_rows;
    t_no_alloc = true;
  }
  ~ScratchView() {
    c->h = h; c->qkv = qkv; c->attn = attn; c->act = act; c->kscr = kscr; c->vscr = vscr; c->xn = xn;
    c->ssq = ssq; c->gpart = gpart; c->apart = apart; c->rope = rope;
    c->gpart_floats = gpart_floats; c->apart_floats = apart_floats; c->rope_floats = rope_floats;
    c->ws_rows = ws_rows;
    t_no_alloc = false;
  }
};

// Largest split-partial need of the four projections at up to NOALLOC_MAX_ROWS rows (fp32 floats).
static size_t noalloc_gemm_partials(const fdllm_ctx* c) {
  const fdllm_config& f = c->cfg;
  size_t need = 0;
  for (int rows = 1; rows <= NOALLOC_MAX_ROWS; ++rows) {
    LayerGemms g = layer_gemms(c, c->layers[0], rows, false);
    const std::pair<int, GemmP*> all[] = {{CFG_QKV, &g.q}, {CFG_OPROJ, &g.o}, {CFG_GATE_UP, &g.gu}, {CFG_DOWN, &g.d}};
    for (const auto& [cfg, a] : all) {
      GemmP t = *a;
      const GemmPlan pl = gemm_plan(cfg, t, cfg == CFG_DOWN ? g.dsplit : 1, c->mm);
      need = std::max(need, pl.part_floats);
    }
  }
  (void)f;
  return need;
}

int fdllm_forward_cached_noalloc(fdllm_ctx* c, const void* x, int rows, void* k, void* v, int cap, const int32_t* off,
                                 int64_t prefix_len, void* out, void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  if (c->scratch_dev == nullptr)
    return fail(FDLLM_EHIP, "the allocation-free step's scratch array is not available on device %d", c->dev);
  if (rows <= 0 || rows > NOALLOC_MAX_ROWS)
    return fail(FDLLM_EINVAL, "the allocation-free step takes 1 .. %d rows, got %d", NOALLOC_MAX_ROWS, rows);
  const fdllm_config& f = c->cfg;
  const size_t R = NOALLOC_MAX_ROWS, H = f.hidden_size, I = f.intermediate_size;
  size_t off_b = 0;
  auto take = [&](size_t bytes) {
    unsigned char* p = c->scratch_dev + off_b;
    off_b += align_up(bytes, 256);
    return p;
  };
  ScratchView keep(c);
  c->h = (uint16_t*)take(R * H * 2);
  c->qkv = (uint16_t*)take(R * c->qkv_dim() * 2);
  c->attn = (uint16_t*)take(R * c->q_dim() * 2);
  c->act = (uint16_t*)take(R * I * 2);
  c->xn = (uint16_t*)take(R * H * 2);
  c->ssq = (float*)take((size_t)c->ssq_tiles() * R * 4);
  c->kscr = c->vscr = nullptr;
  c->ws_rows = (int)R;
  c->rope = (float*)take(R * 128 * 4);
  c->rope_floats = R * 128;
  c->gpart_floats = noalloc_gemm_partials(c);
  c->gpart = (float*)take(c->gpart_floats * 4);
  if (off_b >= NOALLOC_SCRATCH_BYTES)
    return fail(FDLLM_EINVAL, "the model's workspace (%zu bytes) exceeds the allocation-free step's scratch (%zu bytes)",
                off_b, NOALLOC_SCRATCH_BYTES);
  c->apart = (float*)(c->scratch_dev + off_b);
  c->apart_floats = (NOALLOC_SCRATCH_BYTES - off_b) / 4;
  return cached_step(c, x, rows, k, v, cap, off, prefix_len, 0, rows, out, stream);
}

int fdllm_forward_block_partial(fdllm_ctx* c, int rp, const void* x, int rows, void* k, void* v, int cap,
                                const int32_t* off, int64_t prefix_len, void* out, void* stream) {
  if (!c) return fail(FDLLM_EINVAL, "null context");
  const int sbs = c->cfg.bd_size / 4;
  if (rp < 0 || rp % sbs || rp >= c->cfg.bd_size)
    return fail(FDLLM_EINVAL, "replace_position %d is not one of 0, %d, ..., %d", rp, sbs, c->cfg.bd_size - sbs);
  if (rows != sbs) return fail(FDLLM_EINVAL, "partial step takes %d rows, got %d", sbs, rows);
  return cached_step(c, x, rows, k, v, cap, off, prefix_len, rp, c->cfg.bd_size, out, stream);
}

#define FD_PARTIAL(RP)                                                                                     \
  int fdllm_forward_block_partial_rp##RP(fdllm_ctx* c, const void* x, int rows, void* k, void* v, int cap, \
                                         const int32_t* off, int64_t prefix_len, void* out, void* stream) { \
    return fdllm_forward_block_partial(c, RP, x, rows, k, v, cap, off, prefix_len, out, stream);           \
  }
FD_PARTIAL(0)
FD_PARTIAL(8)
FD_PARTIAL(16)
FD_PARTIAL(24)
#undef FD_PARTIAL

// ---- the reference's attention callbacks (fast_dllm_relax/runtime.py:51-80), for a model that computes
// its own projections and RoPE and calls out for the cache write and the attention ----

static int check_kv_call(const fdllm_ctx* c, int rows, int cap, int layer) {
  if (!c) return fail(FDLLM_EINVAL, "null context");
  if (rows < 0) return fail(FDLLM_EINVAL, "rows must not be negative, got %d", rows);
  if (cap <= 0) return fail(FDLLM_EINVAL, "cache capacity must be positive, got %d", cap);
  if (layer < 0 || layer >= c->cfg.num_hidden_layers)
    return fail(FDLLM_EINVAL, "layer %d outside [0, %d)", layer, c->cfg.num_hidden_layers);
  return FDLLM_OK;
}

// _write_rows (runtime.py:51-60): rows [start, start + rows) of the layer's cache get k and v byte for
// byte (a cache row is nkv x head_dim contiguous elements, so the window is one contiguous range).
static int write_kv_rows(const fdllm_ctx* c, const void* k, const void* v, int rows, void* kc, void* vc, int cap,
                         int layer, int64_t start, hipStream_t st) {
  if (start < 0 || start + rows > cap)
    return fail(FDLLM_EINVAL, "KV write [%lld, %lld) outside cache capacity %d", (long long)start,
                (long long)(start + rows), cap);
  if (rows == 0) return FDLLM_OK;
  const size_t row = (size_t)c->cfg.num_key_value_heads * c->cfg.head_dim;
  const size_t off = ((size_t)layer * cap + (size_t)start) * row, bytes = (size_t)rows * row * sizeof(uint16_t);
  uint16_t *kd = (uint16_t*)kc + off, *vd = (uint16_t*)vc + off;
  if (((uintptr_t)k | (uintptr_t)v | (uintptr_t)kd | (uintptr_t)vd | bytes) % 16 == 0 && bytes / 16 <= INT32_MAX) {
    HIPCHK(launch_kv_copy(k, v, kd, vd, bytes, st));  // one launch for both
  } else {
    HIPCHK(hipMemcpyAsync(kd, k, bytes, hipMemcpyDeviceToDevice, st));
    HIPCHK(hipMemcpyAsync(vd, v, bytes, hipMemcpyDeviceToDevice, st));
  }
  return FDLLM_OK;
}

int fdllm_kv_write(fdllm_ctx* c, const void* k, const void* v, int rows, void* k_cache, void* v_cache, int cap,
                   int layer, int64_t start, void* stream) {
  int rc = check_kv_call(c, rows, cap, layer);
  if (rc) return rc;
  if (!k || !v || !k_cache || !v_cache) return fail(FDLLM_EINVAL, "null tensor argument");
  return write_kv_rows(c, k, v, rows, k_cache, v_cache, cap, layer, start, (hipStream_t)stream);
}

// fast_dllm.attn_inplace (runtime.py:63-73): the write of _write_rows, then attention of the given
// (already rotated) queries over cache rows [0, prefix_len + attend_rel) with no mask (_attend,
// runtime.py:30-48).  The chunk and loop kernels take the queries from q (AttnP::rope null: no RoPE, and
// ws = Lk: no rows of the call are read from q's buffer or appended, the cache already holds them); the
// prefill kernels (128 rows and more) read rotated queries from the output buffer, where they are
// copied first.
int fdllm_attn_inplace(fdllm_ctx* c, const void* q, const void* k, const void* v, int rows, void* k_cache,
                       void* v_cache, int cap, int layer, int64_t prefix_len, int write_rel, int attend_rel, void* out,
                       void* stream) {
  int rc = check_kv_call(c, rows, cap, layer);
  if (rc) return rc;
  if (!q || !k || !v || !k_cache || !v_cache || !out) return fail(FDLLM_EINVAL, "null tensor argument");
  rc = check_aligned({q, k_cache, v_cache, out});
  if (rc) return rc;
  const int64_t write_start = prefix_len + write_rel, attend_len = prefix_len + attend_rel;
  if (write_start + rows > attend_len)
    return fail(FDLLM_EINVAL, "KV write [%lld, %lld) past the attended rows [0, %lld)", (long long)write_start,
                (long long)(write_start + rows), (long long)attend_len);
  const hipStream_t st = (hipStream_t)stream;
  rc = write_kv_rows(c, k, v, rows, k_cache, v_cache, cap, layer, write_start, st);
  if (rc || rows == 0) return rc;
  // the reference attends over the slice k_cache[layer, :, :attend_len], which stops at the capacity
  const int Lk = (int)std::min<int64_t>(attend_len, cap);
  const fdllm_config& f = c->cfg;
  const size_t stride = (size_t)cap * f.num_key_value_heads * f.head_dim;
  AttnP a;
  rc = plan_attention(c, a, rows, (uint16_t*)k_cache + layer * stride, (uint16_t*)v_cache + layer * stride, Lk, Lk,
                      0, nullptr, 0, nullptr, false);
  if (rc) return rc;
  a.qkv = (const uint16_t*)q;
  a.ldq = f.num_attention_heads * f.head_dim;
  a.rope = nullptr;
  a.out = (uint16_t*)out;
  if (attn_takes_roped(a)) {
    HIPCHK(hipMemcpyAsync(out, q, (size_t)rows * a.ldq * sizeof(uint16_t), hipMemcpyDeviceToDevice, st));
    a.roped = 1;
  }
  HIPCHK(launch_attention(f.dtype, a, st));
  return FDLLM_OK;
}

int fdllm_forward_cached_batch(fdllm_ctx* c, const void* x, int nseq, int rows, void* k, void* v, int cap,
                               const int32_t* off, const int64_t* prefix_lens, void* out, void* stream) {
  return cached_step_batch(c, x, nseq, rows, k, v, cap, off, prefix_lens, 0, rows, out, stream);
}

int fdllm_forward_block_partial_batch(fdllm_ctx* c, int rp, const void* x, int nseq, int rows, void* k, void* v,
                                      int cap, const int32_t* off, const int64_t* prefix_lens, void* out,
                                      void* stream) {
  if (!c) return fail(FDLLM_EINVAL, "null context");
  const int sbs = c->cfg.bd_size / 4;
  if (rp < 0 || rp % sbs || rp >= c->cfg.bd_size)
    return fail(FDLLM_EINVAL, "replace_position %d is not one of 0, %d, ..., %d", rp, sbs, c->cfg.bd_size - sbs);
  if (rows != sbs) return fail(FDLLM_EINVAL, "partial step takes %d rows, got %d", sbs, rows);
  return cached_step_batch(c, x, nseq, rows, k, v, cap, off, prefix_lens, rp, c->cfg.bd_size, out, stream);
}

int fdllm_build_prefix_cache_seq(fdllm_ctx* c, const void* x, int P, const float* bias, void* k, void* v, int cap,
                                 int nseq, int seq, void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  rc = pending_wait_fault(c);
  if (rc) return rc;
  if (P <= 0 || !x || !k || !v) return fail(FDLLM_EINVAL, "invalid build_prefix_cache arguments");
  rc = check_aligned({x, k, v});
  if (rc) return rc;
  if (nseq <= 0 || seq < 0 || seq >= nseq) return fail(FDLLM_EINVAL, "sequence %d of a batch of %d", seq, nseq);
  if (P > cap) return fail(FDLLM_EINVAL, "KV write [0, %d) outside cache capacity %d", P, cap);
  rc = ensure_rows(c, P);
  if (rc) return rc;
  const fdllm_config& f = c->cfg;
  const size_t seq_stride = (size_t)cap * f.num_key_value_heads * f.head_dim;
  uint16_t* kb = (uint16_t*)k + (size_t)seq * seq_stride;
  uint16_t* vb = (uint16_t*)v + (size_t)seq * seq_stride;
  return run_layers(c, x, P, kb, vb, (size_t)nseq * seq_stride, 0, c->zero_i32, P, bias ? 2 : 1, bias, P, nullptr,
                    (hipStream_t)stream);
}

int fdllm_get_confidence(fdllm_ctx* c, const void* hidden, int rows, int32_t* ids, float* maxp, float* logits,
                         void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  rc = pending_wait_fault(c);
  if (rc) return rc;
  if (rows <= 0 || !hidden || !ids || !maxp) return fail(FDLLM_EINVAL, "invalid get_confidence arguments");
  rc = check_aligned({hidden, logits});
  if (rc) return rc;
  rc = ensure_stats(c, rows);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  rc = run_lm_head(c, (const uint16_t*)hidden, rows, logits, true, st);
  if (rc) return rc;
  int T = c->tiles();
  char* base = (char*)c->stats;
  HIPCHK(launch_confidence_combine((float*)base, (int32_t*)(base + c->stats_rows * T * 4),
                                   (float*)(base + c->stats_rows * T * 8), T, rows, ids, maxp, st));
  return FDLLM_OK;
}

// The sub-block arguments of the unmask entry points (block rows [s0, s0 + sub) take confidence rows
// [row0, row0 + sub) after the shift).
static int check_unmask(const fdllm_ctx* c, int rows, int row0, const int32_t* block, int s0, int sub,
                        float threshold) {
  const int bd = c->cfg.bd_size;
  if (!block) return fail(FDLLM_EINVAL, "null block");
  if (bd > 64) return fail(FDLLM_EINVAL, "the device unmask takes blocks of at most 64 rows (bd_size %d)", bd);
  if (rows <= 0) return fail(FDLLM_EINVAL, "confidence rows must be positive, got %d", rows);
  if (sub < 0 || s0 < 0 || s0 + sub > bd)
    return fail(FDLLM_EINVAL, "sub-block [%d, %d) outside the block of %d rows", s0, s0 + sub, bd);
  if (row0 < 0 || row0 + sub > rows)
    return fail(FDLLM_EINVAL, "confidence rows [%d, %d) outside the call's %d rows", row0, row0 + sub, rows);
  if (!(threshold == threshold)) return fail(FDLLM_EINVAL, "threshold is NaN");
  return FDLLM_OK;
}

static UnmaskP unmask_args(const fdllm_ctx* c, int rows, int row0, int32_t* block, int s0, int sub, int32_t mask_id,
                           float threshold, int32_t* report, int32_t seq) {
  UnmaskP u{};
  u.rows = rows; u.row0 = row0; u.block = block; u.bd = c->cfg.bd_size; u.s0 = s0; u.sub = sub;
  u.mask_id = mask_id; u.thr = threshold; u.report = report; u.seq = seq;
  return u;
}

int fdllm_unmask(fdllm_ctx* c, const int32_t* ids, const float* maxp, int rows, int row0, int32_t* block, int s0,
                 int sub_rows, int32_t mask_id, float threshold, int32_t* report, int32_t seq, void* stream) {
  if (!c) return fail(FDLLM_EINVAL, "null context");
  int rc = pending_wait_fault(c);
  if (rc) return rc;
  if (!ids || !maxp) return fail(FDLLM_EINVAL, "null confidence argument");
  rc = check_unmask(c, rows, row0, block, s0, sub_rows, threshold);
  if (rc) return rc;
  HIPCHK(launch_unmask(ids, maxp, unmask_args(c, rows, row0, block, s0, sub_rows, mask_id, threshold, report, seq),
                       (hipStream_t)stream));
  return FDLLM_OK;
}

int fdllm_get_confidence_unmask(fdllm_ctx* c, const void* hidden, int rows, int row0, int32_t* block, int s0,
                                int sub_rows, int32_t mask_id, float threshold, int32_t* ids, float* maxp,
                                int32_t* report, int32_t seq, void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  rc = pending_wait_fault(c);
  if (rc) return rc;
  if (!hidden) return fail(FDLLM_EINVAL, "null hidden states");
  rc = check_aligned({hidden});
  if (rc) return rc;
  if ((ids == nullptr) != (maxp == nullptr)) return fail(FDLLM_EINVAL, "ids and maxp must both be given or both be null");
  rc = check_unmask(c, rows, row0, block, s0, sub_rows, threshold);
  if (rc) return rc;
  if (rows > 1024) return fail(FDLLM_EINVAL, "the fused unmask combines at most 1024 rows, got %d", rows);
  rc = ensure_stats(c, rows);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  rc = run_lm_head(c, (const uint16_t*)hidden, rows, nullptr, true, st);
  if (rc) return rc;
  const int T = c->tiles();
  char* base = (char*)c->stats;
  HIPCHK(launch_confidence_unmask((float*)base, (int32_t*)(base + c->stats_rows * T * 4),
                                  (float*)(base + c->stats_rows * T * 8), T, (int)c->stats_rows, ids, maxp,
                                  unmask_args(c, rows, row0, block, s0, sub_rows, mask_id, threshold, report, seq), st));
  return FDLLM_OK;
}

int fdllm_host_alloc(size_t bytes, void** host_ptr, void** device_ptr) {
  if (!host_ptr || !device_ptr || bytes == 0) return fail(FDLLM_EINVAL, "invalid host_alloc arguments");
  *host_ptr = *device_ptr = nullptr;
  HIPCHK(hipHostMalloc(host_ptr, bytes, hipHostMallocMapped | hipHostMallocCoherent));
  std::memset(*host_ptr, 0, bytes);
  const hipError_t e = hipHostGetDevicePointer(device_ptr, *host_ptr, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(*host_ptr);
    *host_ptr = nullptr;
    return fail(FDLLM_EHIP, "hipHostGetDevicePointer: %s", hipGetErrorString(e));
  }
  return FDLLM_OK;
}

void fdllm_host_free(void* host_ptr) {
  if (host_ptr) (void)hipHostFree(host_ptr);
}

long long fdllm_group_wait_launches(const fdllm_ctx* c) { return c ? c->group_wait_launches : 0; }

long long fdllm_frag_calls(const fdllm_ctx* c) { return c ? c->frag_calls : 0; }

int fdllm_bench_op(fdllm_ctx* c, int op, int rows, int layer, int iters, void* k, void* v, int cap, int attend_len,
                   void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  const fdllm_config& f = c->cfg;
  if (rows <= 0 || iters <= 0 || layer < 0 || layer >= f.num_hidden_layers)
    return fail(FDLLM_EINVAL, "invalid bench_op arguments");
  if (op == FDLLM_OP_ATTENTION && (!k || !v || attend_len < rows || attend_len > cap))
    return fail(FDLLM_EINVAL, "attention needs a cache holding attend_len >= rows rows");
  rc = ensure_rows(c, rows);
  if (rc == FDLLM_OK) rc = ensure_stats(c, rows);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  const size_t stride = (size_t)cap * f.num_key_value_heads * f.head_dim;
  // the launches a cached step of `rows` rows makes (layout included), on whatever the buffers hold
  const bool frag = frag_chain(c, rows);
  for (int it = 0; it < iters && rc == FDLLM_OK; ++it) {
    // consecutive launches walk the layers, as a step does, so no weight is re-read from cache
    const int li = (layer + it) % f.num_hidden_layers;
    LayerGemms g = layer_gemms(c, c->layers[li], rows, frag);
    switch (op) {
      case FDLLM_OP_QKV: rc = run_gemm(c, CFG_QKV, g.q, 1, st); break;
      case FDLLM_OP_O_PROJ: rc = run_gemm(c, CFG_OPROJ, g.o, 1, st); break;
      case FDLLM_OP_GATE_UP: rc = run_gemm(c, CFG_GATE_UP, g.gu, 1, st); break;
      case FDLLM_OP_DOWN: rc = run_gemm(c, CFG_DOWN, g.d, g.dsplit, st); break;
      case FDLLM_OP_ATTENTION:
        // the block's rows sit at the end of the attended range, as in a full cached step
        if (it == 0) rc = rope_table(c, rows, c->zero_i32, rows, st);
        if (rc == FDLLM_OK)
          rc = run_attention(c, rows, (uint16_t*)k + li * stride, (uint16_t*)v + li * stride, attend_len - rows,
                             attend_len, 0, nullptr, 0, st, nullptr, frag);
        break;
      case FDLLM_OP_LM_HEAD_CONFIDENCE: {
        rc = run_lm_head(c, c->h, rows, nullptr, true, st);
        if (rc) break;
        const int T = c->tiles();
        char* base = (char*)c->stats;
        int32_t* ids = (int32_t*)c->qkv;
        float* maxp = (float*)(c->qkv + 64);
        HIPCHK(launch_confidence_combine((float*)base, (int32_t*)(base + c->stats_rows * T * 4),
                                         (float*)(base + c->stats_rows * T * 8), T, rows, ids, maxp, st));
        break;
      }
      default:
        return fail(FDLLM_EINVAL, "unknown op %d", op);
    }
  }
  return rc;
}

int fdllm_confidence_from_logits(fdllm_ctx* c, const float* logits, int rows, int vocab, int ld, int32_t* ids,
                                 float* maxp, void* stream) {
  if (!c) return fail(FDLLM_EINVAL, "null context");
  if (rows <= 0 || vocab <= 0 || ld < vocab || !logits || !ids || !maxp)
    return fail(FDLLM_EINVAL, "invalid confidence arguments");
  if (vocab != c->cfg.vocab_size) return fail(FDLLM_EINVAL, "vocab %d differs from the model's %d", vocab, c->cfg.vocab_size);
  int rc = ensure_stats(c, rows);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  int T = c->tiles();
  char* base = (char*)c->stats;
  float* sm = (float*)base;
  int32_t* sa = (int32_t*)(base + c->stats_rows * T * 4);
  float* ss = (float*)(base + c->stats_rows * T * 8);
  HIPCHK(launch_confidence_tiles(logits, ld, vocab, rows, sm, sa, ss, st));
  HIPCHK(launch_confidence_combine(sm, sa, ss, T, rows, ids, maxp, st));
  return FDLLM_OK;
}

}  // extern "C"
