// C ABI: context, weight binding, workspace, launch planning and the nine entry points.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "../../include/fdllm.h"
#include "kernels.hpp"

using namespace fdllm;

namespace {

thread_local std::string g_err;

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
  const uint16_t *wqkv, *bqkv, *wo, *wgu, *wd, *ln_in, *ln_post;
};

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

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

  // row workspace (grown on demand)
  int ws_rows = 0;
  void* ws = nullptr;
  uint16_t *h = nullptr, *xn = nullptr, *qkv = nullptr, *qrot = nullptr, *attn = nullptr, *act = nullptr;
  uint16_t *kscr = nullptr, *vscr = nullptr;  // K/V of a stateless forward (one layer at a time)
  // split-K partials / attention partials / confidence statistics (grown on demand)
  float* gpart = nullptr; size_t gpart_floats = 0;
  float* apart = nullptr; size_t apart_floats = 0;
  void* stats = nullptr; size_t stats_rows = 0;
  int* counters = nullptr; int n_counters = 0;
  int32_t* zero_i32 = nullptr;
  int wg_target = 256;

  int qkv_dim() const { return (cfg.num_attention_heads + 2 * cfg.num_key_value_heads) * cfg.head_dim; }
  int q_dim() const { return cfg.num_attention_heads * cfg.head_dim; }
  int kv_dim() const { return cfg.num_key_value_heads * cfg.head_dim; }
  int tiles() const { return (cfg.vocab_size + 255) / 256; }
};

namespace {

int ensure_rows(fdllm_ctx* c, int rows) {
  if (rows <= c->ws_rows) return FDLLM_OK;
  int R = (int)align_up((size_t)std::max(rows, 32), 32);
  const fdllm_config& f = c->cfg;
  size_t e_h = (size_t)R * f.hidden_size, e_qkv = (size_t)R * c->qkv_dim(), e_q = (size_t)R * c->q_dim();
  size_t e_act = (size_t)R * f.intermediate_size, e_kv = (size_t)R * c->kv_dim();
  size_t bytes = 2 * (align_up(e_h, 64) * 2 + align_up(e_qkv, 64) + align_up(e_q, 64) * 2 + align_up(e_act, 64) +
                      align_up(e_kv, 64) * 2);
  if (c->ws) HIPCHK(hipFree(c->ws));
  c->ws = nullptr;
  HIPCHK(hipMalloc(&c->ws, bytes));
  uint16_t* p = (uint16_t*)c->ws;
  auto take = [&](size_t n) { uint16_t* r = p; p += align_up(n, 64); return r; };
  c->h = take(e_h); c->xn = take(e_h); c->qkv = take(e_qkv); c->qrot = take(e_q); c->attn = take(e_q);
  c->act = take(e_act); c->kscr = take(e_kv); c->vscr = take(e_kv);
  c->ws_rows = R;
  return FDLLM_OK;
}

int ensure_floats(float** buf, size_t* have, size_t need) {
  if (need <= *have) return FDLLM_OK;
  if (*buf) HIPCHK(hipFree(*buf));
  *buf = nullptr;
  size_t n = align_up(need, 1 << 20);
  HIPCHK(hipMalloc((void**)buf, n * sizeof(float)));
  *have = n;
  return FDLLM_OK;
}

int ensure_stats(fdllm_ctx* c, int rows) {
  if ((size_t)rows <= c->stats_rows) return FDLLM_OK;
  size_t R = align_up((size_t)std::max(rows, 32), 32);
  if (c->stats) HIPCHK(hipFree(c->stats));
  c->stats = nullptr;
  HIPCHK(hipMalloc(&c->stats, R * c->tiles() * 12));
  c->stats_rows = R;
  return FDLLM_OK;
}

// ---- launch planning -----------------------------------------------------------------------------
struct Plan {
  int tpw, mt, nblocks, ksplit, mchunks, kc, wg_rows, tile_stride;
};

Plan plan_gemm(const fdllm_ctx* c, int M, int N, int K, int epi) {
  Plan p{};
  p.mt = M <= 16 ? 1 : 2;
  p.mchunks = (M + 16 * p.mt - 1) / (16 * p.mt);
  if (epi == EPI_SILU) {
    p.tpw = 2; p.wg_rows = 64; p.tile_stride = N / 2; p.nblocks = (N / 2 + 63) / 64;
  } else if (epi == EPI_LOGITS) {
    p.tpw = 4; p.wg_rows = 256; p.tile_stride = 64; p.nblocks = (N + 255) / 256;
  } else {
    p.tpw = 2; p.wg_rows = 128; p.tile_stride = 64; p.nblocks = (N + 127) / 128;
  }
  if (epi == EPI_LOGITS) {  // one workgroup per 256-column confidence tile, whole K in LDS
    p.ksplit = 1;
    p.kc = K;
    return p;
  }
  const int steps = K / 128;
  int best = -1;
  long best_cost = 0;
  for (int d = 1; d <= steps; ++d) {
    if (steps % d) continue;
    int kc = K / d;
    if (kc > 1024) continue;
    long total = (long)p.nblocks * p.mchunks * d;
    long cost = std::labs(total - c->wg_target) + (d > 1 ? (long)d * 4 : 0);
    if (best < 0 || cost < best_cost) { best = d; best_cost = cost; }
  }
  p.ksplit = best < 0 ? 1 : best;
  p.kc = K / p.ksplit;
  return p;
}

int run_gemm(fdllm_ctx* c, int epi, const uint16_t* X, int ldx, int M, const uint16_t* W, int N, int K,
             uint16_t* Y, int ldy, const uint16_t* bias, const uint16_t* resid, int ldr, float* logits, int ldl,
             bool stats, hipStream_t st) {
  if (K % 128 != 0) return fail(FDLLM_EINVAL, "GEMM K=%d is not a multiple of 128", K);
  Plan p = plan_gemm(c, M, N, K, epi);
  if (epi == EPI_LOGITS && p.kc > 2048) return fail(FDLLM_EINVAL, "hidden size %d too large for the lm_head kernel", K);
  GemmArgs a{};
  a.X = X; a.ldx = ldx; a.M = M; a.W = W; a.N = N; a.K = K; a.kc = p.kc;
  a.wg_rows = p.wg_rows; a.tile_stride = p.tile_stride;
  a.Y = Y; a.ldy = ldy; a.bias = bias; a.resid = resid; a.ldr = ldr; a.logits = logits; a.ldl = ldl;
  if (p.ksplit > 1) {
    size_t need = (size_t)p.nblocks * p.mchunks * p.ksplit * 4 * p.tpw * p.mt * 64 * 4;
    int rc = ensure_floats(&c->gpart, &c->gpart_floats, need);
    if (rc) return rc;
    if (p.nblocks * p.mchunks > c->n_counters) return fail(FDLLM_EINVAL, "too many GEMM column blocks (%d)", p.nblocks * p.mchunks);
    a.partial = c->gpart;
    a.counters = c->counters;
  }
  if (stats) {
    int T = c->tiles();
    char* base = (char*)c->stats;
    a.stat_m = (float*)base;
    a.stat_a = (int32_t*)(base + c->stats_rows * T * 4);
    a.stat_s = (float*)(base + c->stats_rows * T * 8);
    a.stat_tiles = T;
  }
  HIPCHK(launch_gemm(c->cfg.dtype, epi, p.tpw, p.mt, a, p.nblocks, p.ksplit, p.mchunks, st));
  return FDLLM_OK;
}

int run_attention(fdllm_ctx* c, int rows, const uint16_t* kc, const uint16_t* vc, int Lk, int mask, int q_pos0,
                  const float* bias, long long bias_ld, hipStream_t st) {
  const fdllm_config& f = c->cfg;
  AttnArgs a{};
  a.q = c->qrot; a.k = kc; a.v = vc;
  a.rows = rows; a.nq = f.num_attention_heads; a.nkv = f.num_key_value_heads; a.hd = f.head_dim;
  a.Lk = Lk; a.scale = 1.0f / std::sqrt((float)f.head_dim);
  a.mask = mask; a.q_pos0 = q_pos0; a.block = f.bd_size; a.bias = bias; a.bias_ld = bias_ld;
  const int grp = a.nq / a.nkv;
  const int QR = grp * rows;
  const int qtiles = (QR + 15) / 16;
  const int nqg = (qtiles + 3) / 4;
  a.QRp = qtiles * 16;
  int base = nqg * a.nkv;
  int nsplit = std::max(1, std::min((c->wg_target + base - 1) / base, (Lk + 255) / 256));
  int chunk = (int)align_up((size_t)((Lk + nsplit - 1) / nsplit), 64);
  nsplit = (Lk + chunk - 1) / chunk;
  a.nsplit = nsplit; a.chunk = chunk;
  size_t per = (size_t)nsplit * a.nkv * a.QRp;
  int rc = ensure_floats(&c->apart, &c->apart_floats, per * (a.hd + 2));
  if (rc) return rc;
  a.o_part = c->apart; a.m_part = c->apart + per * a.hd; a.l_part = a.m_part + per;
  a.out = c->attn;
  HIPCHK(launch_attention(f.dtype, a, nqg, st));
  return FDLLM_OK;
}

// The decoder-layer loop (cuda.py:561-579 per layer, 639-666 for the model).
// kv: per-layer cache base pointers come from k/v + layer * layer_stride (elements).
int run_layers(fdllm_ctx* c, const void* x_in, int rows, uint16_t* kbase, uint16_t* vbase, size_t layer_stride,
               int write_start, const int32_t* pos_dev, int attend_len, int mask, const float* bias,
               long long bias_ld, void* out, hipStream_t st) {
  const fdllm_config& f = c->cfg;
  const int H = f.hidden_size, I = f.intermediate_size;
  HIPCHK(hipMemcpyAsync(c->h, x_in, (size_t)rows * H * 2, hipMemcpyDeviceToDevice, st));
  for (int l = 0; l < f.num_hidden_layers; ++l) {
    const Layer& L = c->layers[l];
    uint16_t* kc = kbase + (size_t)l * layer_stride;
    uint16_t* vc = vbase + (size_t)l * layer_stride;
    HIPCHK(launch_rmsnorm(f.dtype, c->h, H, rows, H, L.ln_in, f.rms_norm_eps, c->xn, H, st));
    int rc = run_gemm(c, EPI_BIAS, c->xn, H, rows, L.wqkv, c->qkv_dim(), H, c->qkv, c->qkv_dim(), L.bqkv, nullptr, 0,
                      nullptr, 0, false, st);
    if (rc) return rc;
    RopeArgs ra{};
    ra.qkv = c->qkv; ra.ld = c->qkv_dim(); ra.rows = rows; ra.nq = f.num_attention_heads;
    ra.nkv = f.num_key_value_heads; ra.hd = f.head_dim; ra.pos_offset = pos_dev;
    ra.neg_log_theta = (float)(-std::log((double)f.rope_theta));
    ra.q_out = c->qrot; ra.k_cache = kc; ra.v_cache = vc; ra.write_start = write_start;
    HIPCHK(launch_rope_kv(f.dtype, ra, st));
    rc = run_attention(c, rows, kc, vc, attend_len, mask, 0, bias, bias_ld, st);
    if (rc) return rc;
    rc = run_gemm(c, EPI_RESID, c->attn, c->q_dim(), rows, L.wo, H, c->q_dim(), c->h, H, nullptr, c->h, H, nullptr, 0,
                  false, st);
    if (rc) return rc;
    HIPCHK(launch_rmsnorm(f.dtype, c->h, H, rows, H, L.ln_post, f.rms_norm_eps, c->xn, H, st));
    rc = run_gemm(c, EPI_SILU, c->xn, H, rows, L.wgu, 2 * I, H, c->act, I, nullptr, nullptr, 0, nullptr, 0, false, st);
    if (rc) return rc;
    rc = run_gemm(c, EPI_RESID, c->act, I, rows, L.wd, H, I, c->h, H, nullptr, c->h, H, nullptr, 0, false, st);
    if (rc) return rc;
  }
  HIPCHK(launch_rmsnorm(f.dtype, c->h, H, rows, H, c->final_norm, f.rms_norm_eps, (uint16_t*)out, H, st));
  return FDLLM_OK;
}

int check_ready(const fdllm_ctx* c) {
  if (!c) return fail(FDLLM_EINVAL, "null context");
  if (!c->bound) return fail(FDLLM_ESTATE, "weights are not bound (fdllm_bind_weights)");
  return FDLLM_OK;
}

int cached_step(fdllm_ctx* c, const void* x, int rows, void* k, void* v, int cap, const int32_t* off,
                int64_t prefix_len, int write_rel, int attend_rel, void* out, void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  if (!x || !k || !v || !off || !out) return fail(FDLLM_EINVAL, "null tensor argument");
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
  if (const char* e = std::getenv("FDLLM_WG_TARGET")) c->wg_target = std::max(1, atoi(e));
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
  hipError_t e = hipMalloc((void**)&c->counters, (size_t)c->n_counters * 4 + 64);
  if (e == hipSuccess) e = hipMemset(c->counters, 0, (size_t)c->n_counters * 4 + 64);
  if (e != hipSuccess) {
    delete c;
    return fail(FDLLM_EHIP, "workspace allocation failed: %s", hipGetErrorString(e));
  }
  c->zero_i32 = (int32_t*)(c->counters + c->n_counters);
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
  for (void* p : {c->ws, (void*)c->gpart, (void*)c->apart, c->stats, (void*)c->counters})
    if (p) (void)hipFree(p);
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
  for (int i = 0; i < n; ++i)
    if (!ptrs[i]) return fail(FDLLM_EINVAL, "param %d (%s) is null", i, c->names[i].c_str());
  c->params.assign((const uint16_t* const*)ptrs, (const uint16_t* const*)ptrs + n);
  c->embed = c->params[0];
  c->layers.resize(c->cfg.num_hidden_layers);
  for (int i = 0; i < c->cfg.num_hidden_layers; ++i) {
    const uint16_t* const* p = &c->params[1 + 7 * i];
    c->layers[i] = Layer{p[0], p[1], p[2], p[3], p[4], p[5], p[6]};
  }
  c->final_norm = c->params[1 + 7 * c->cfg.num_hidden_layers];
  c->lm_head = c->cfg.tie_word_embeddings ? c->embed : c->params[2 + 7 * c->cfg.num_hidden_layers];
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
  if (S <= 0) return fail(FDLLM_EINVAL, "seq_len must be positive, got %d", S);
  if (!x || !out) return fail(FDLLM_EINVAL, "null tensor argument");
  rc = ensure_rows(c, S);
  if (rc) return rc;
  return run_layers(c, x, S, c->kscr, c->vscr, 0, 0, c->zero_i32, S, bias ? 2 : 1, bias, S, out, (hipStream_t)stream);
}

int fdllm_get_logits(fdllm_ctx* c, const void* hidden, int rows, float* logits, void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  if (rows <= 0 || !hidden || !logits) return fail(FDLLM_EINVAL, "invalid get_logits arguments");
  const fdllm_config& f = c->cfg;
  return run_gemm(c, EPI_LOGITS, (const uint16_t*)hidden, f.hidden_size, rows, c->lm_head, f.vocab_size,
                  f.hidden_size, nullptr, 0, nullptr, nullptr, 0, logits, f.vocab_size, false, (hipStream_t)stream);
}

int fdllm_build_prefix_cache(fdllm_ctx* c, const void* x, int P, const float* bias, void* k, void* v, int cap,
                             void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  if (P <= 0 || !x || !k || !v) return fail(FDLLM_EINVAL, "invalid build_prefix_cache arguments");
  if (P > cap) return fail(FDLLM_EINVAL, "KV write [0, %d) outside cache capacity %d", P, cap);
  rc = ensure_rows(c, P);
  if (rc) return rc;
  const fdllm_config& f = c->cfg;
  size_t stride = (size_t)cap * f.num_key_value_heads * f.head_dim;
  // build_prefix_cache returns only the caches; the final hidden goes to scratch
  return run_layers(c, x, P, (uint16_t*)k, (uint16_t*)v, stride, 0, c->zero_i32, P, bias ? 2 : 1, bias, P, c->xn,
                    (hipStream_t)stream);
}

int fdllm_forward_cached(fdllm_ctx* c, const void* x, int rows, void* k, void* v, int cap, const int32_t* off,
                         int64_t prefix_len, void* out, void* stream) {
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

int fdllm_get_confidence(fdllm_ctx* c, const void* hidden, int rows, int32_t* ids, float* maxp, float* logits,
                         void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  if (rows <= 0 || !hidden || !ids || !maxp) return fail(FDLLM_EINVAL, "invalid get_confidence arguments");
  rc = ensure_stats(c, rows);
  if (rc) return rc;
  const fdllm_config& f = c->cfg;
  hipStream_t st = (hipStream_t)stream;
  rc = run_gemm(c, EPI_LOGITS, (const uint16_t*)hidden, f.hidden_size, rows, c->lm_head, f.vocab_size, f.hidden_size,
                nullptr, 0, nullptr, nullptr, 0, logits, f.vocab_size, true, st);
  if (rc) return rc;
  int T = c->tiles();
  char* base = (char*)c->stats;
  HIPCHK(launch_confidence_combine((float*)base, (int32_t*)(base + c->stats_rows * T * 4),
                                   (float*)(base + c->stats_rows * T * 8), T, rows, ids, maxp, st));
  return FDLLM_OK;
}

int fdllm_bench_op(fdllm_ctx* c, int op, int rows, int layer, int iters, void* k, void* v, int cap, int attend_len,
                   void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  const fdllm_config& f = c->cfg;
  if (rows <= 0 || iters <= 0 || layer < 0 || layer >= f.num_hidden_layers)
    return fail(FDLLM_EINVAL, "invalid bench_op arguments");
  rc = ensure_rows(c, rows);
  if (rc == FDLLM_OK) rc = ensure_stats(c, rows);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int H = f.hidden_size, I = f.intermediate_size;
  for (int it = 0; it < iters && rc == FDLLM_OK; ++it) {
    // consecutive launches walk the layers, as a step does, so no weight is re-read from cache
    const int li = (layer + it) % f.num_hidden_layers;
    const Layer& L = c->layers[li];
    switch (op) {
      case FDLLM_OP_QKV:
        rc = run_gemm(c, EPI_BIAS, c->xn, H, rows, L.wqkv, c->qkv_dim(), H, c->qkv, c->qkv_dim(), L.bqkv, nullptr, 0,
                      nullptr, 0, false, st);
        break;
      case FDLLM_OP_O_PROJ:
        rc = run_gemm(c, EPI_RESID, c->attn, c->q_dim(), rows, L.wo, H, c->q_dim(), c->h, H, nullptr, c->h, H, nullptr,
                      0, false, st);
        break;
      case FDLLM_OP_GATE_UP:
        rc = run_gemm(c, EPI_SILU, c->xn, H, rows, L.wgu, 2 * I, H, c->act, I, nullptr, nullptr, 0, nullptr, 0, false,
                      st);
        break;
      case FDLLM_OP_DOWN:
        rc = run_gemm(c, EPI_RESID, c->act, I, rows, L.wd, H, I, c->h, H, nullptr, c->h, H, nullptr, 0, false, st);
        break;
      case FDLLM_OP_ATTENTION: {
        if (!k || !v || attend_len <= 0 || attend_len > cap) return fail(FDLLM_EINVAL, "attention needs a cache");
        size_t stride = (size_t)cap * f.num_key_value_heads * f.head_dim;
        rc = run_attention(c, rows, (uint16_t*)k + (size_t)li * stride, (uint16_t*)v + (size_t)li * stride,
                           attend_len, 0, 0, nullptr, 0, st);
        break;
      }
      case FDLLM_OP_LM_HEAD_CONFIDENCE: {
        rc = run_gemm(c, EPI_LOGITS, c->xn, H, rows, c->lm_head, f.vocab_size, H, nullptr, 0, nullptr, nullptr, 0,
                      nullptr, f.vocab_size, true, st);
        if (rc) break;
        int T = c->tiles();
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
