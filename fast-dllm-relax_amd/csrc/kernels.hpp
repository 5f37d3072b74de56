// Kernel launch interfaces shared by the C ABI (capi.hip) and the kernel files.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fdllm {

// ---- packed weights ----------------------------------------------------------------------------
// A weight matrix W [N, K] (nn.Linear layout) is repacked once, at bind time, into MFMA fragment
// order: tile t (16 rows), k step s (32 columns) is one contiguous 1 KB block in which lane l holds
// W[16 t + l % 16][32 s + 8 (l / 16) .. + 8].  A wave then streams whole 1 KB blocks with one
// coalesced load each.  Tiles past the last row are zero.  PACK_PAIRS interleaves the two halves of
// the fused gate_up matrix: packed tile 2p = gate rows [16p, 16p + 16), tile 2p + 1 = the matching
// up rows [I + 16p, ...), so one wave holds both operands of the SiLU * up product.
enum PackMode : int { PACK_ROWS = 0, PACK_PAIRS = 1 };
hipError_t launch_pack(const uint16_t* src, int N, int K, int ntiles, int mode, uint16_t* dst, hipStream_t st);

// ---- workgroups of one launch waiting on each other ----------------------------------------------
// The one-shot projections' k splits (down) are reduced inside their own launch: the
// workgroups of a group store their fp32 partials with agent-scope stores, count their arrival on the
// group's counter and wait until the group's last member has arrived; then each sums a share of the
// group's outputs.  Such a launch is planned only when its whole grid is resident at once (at most one
// workgroup per compute unit), so every member of a group runs.  Every wait is still bounded: past
// `limit` ticks of the 100 MHz wall clock a workgroup gives up, sets *fault (pinned host memory,
// written with a system-scope store) and skips its share, so a broken launch ends with a reported
// fault instead of a hung GPU.
// Counters: two banks of GW_GROUPS counters GW_STRIDE words apart (group k of bank b at
// (b GW_GROUPS + k) GW_STRIDE).  Launches that use a region alternate banks; each launch's workgroup i
// zeroes counter i of the other bank, for i < clear (the groups the previous launch used), since that
// launch has finished (launches of a context are stream-ordered).  So no arrival has to return a value
// and nothing is reset on a wait's critical path.
constexpr int GW_STRIDE = 32;
constexpr int GW_GROUPS = 256;  // groups of one launch (counters in each bank)
struct GroupWait {
  unsigned* cnt;      // the region's two banks; nullptr: the launch reduces with a separate kernel
  unsigned* fault;    // device address of the host-visible fault word
  long long limit;    // wall-clock ticks one wait may take
  int bank;           // bank of this launch
  int clear;          // counters of the other bank to zero
};

constexpr int MAX_SEQS = 64;  // sequences of one batched call

// ---- skinny GEMM over packed weights ------------------------------------------------------------
// Y[M, N] = X[M, K] . W[N, K]^T for M <= 32 per m-chunk (gridDim.z chunks of 32 rows).
enum Epilogue : int { EPI_BIAS = 0, EPI_RESID = 1, EPI_SILU_PAIR = 2, EPI_LOGITS = 3 };
enum XForm : int { XF_NONE = 0, XF_RMS = 1 };

// The qkv projection of a call whose attention takes its queries and new keys already RoPE'd (the
// prefill and batched-sequence kernels, which otherwise start with rope_kv_kernel): its epilogue applies
// rope_kv_kernel's arithmetic (bias, rounding, RoPE of the q and k heads from the table rope, [rows][64][2])
// and writes the q heads to q ([rows][nq x 128]) and the k / v heads of row r of sequence b = r / rows to
// the cache rows ws[b] + r % rows of kc / vc + b seq_stride ([cap][nkv][128]), instead of Y.  The
// register-weight kernel then takes its 16-column tiles in the order perm8 (each head's tiles 0, 1, 4, 5,
// 2, 3, 6, 7), so that the two halves of every rotation pair sit in one wave or in two waves of one block.
struct RopeOut {
  const float* rope; uint16_t* q; uint16_t* kc; uint16_t* vc;
  int nq, nkv, rows; long long seq_stride;
  int ws[MAX_SEQS];
};
__host__ __device__ constexpr int perm8(int t) { return (t & ~6) | ((t & 2) << 1) | ((t & 4) >> 1); }

struct GemmP {
  const uint16_t* W; int KS;          // packed weights, k steps (K / 32)
  int ntiles;                         // packed tiles (the launch covers them all)
  int N;                              // output columns written (rows of W; gate_up: I)
  const uint16_t* X; int ldx; int M;  // activations [M][ldx]
  int kps;                            // k steps per cross-workgroup split (KS / gridDim.y)
  // XF_RMS: X is normalized on the fly with inv_rms[m] = 1 / sqrt(sum_t ssq[t][m] / H + eps)
  const float* ssq; int ssq_tiles; int ssq_ld; const uint16_t* nw; float eps; int H;
  uint16_t* Y; int ldy;               // EPI_BIAS / EPI_SILU_PAIR output
  const uint16_t* bias;               // EPI_BIAS
  float* ssq_out;                     // EPI_RESID: Y (= h, updated in place) + per-tile row sums of squares
  float* logits; int ldl;             // EPI_LOGITS (optional)
  float* stat_m; int32_t* stat_a; float* stat_s; int stat_tiles;  // EPI_LOGITS confidence statistics
  float* part; unsigned* counters;    // cross-workgroup split partials / arrival counters
  int ngroups;                        // tile groups of the one-shot and streaming launches
  // streaming kernel, one gridDim.y: column groups tail_full .. ngroups - 1 each split k tail_split ways
  // over workgroups tail_full + tail_split (group - tail_full) + split (tail_split <= 1: no tail split)
  int tail_full, tail_split;
  // 1: one-shot chains (M <= 32, the register-fragment body only): X, and Y of EPI_RESID /
  // EPI_SILU_PAIR, in MFMA-fragment order (frag_off) instead of row-major; 2: X, and the Y of
  // EPI_SILU_PAIR, in the large-M LDS-staged kernel's fragment blocks (frag_blk_off)
  int xfrag, yfrag;
  // large-M k splits: 1 stores the split sums row-major (part[split][M][N], N a multiple of 4) and launches
  // no split-sum kernel; the caller sums them (launch_resid_norm)
  int part_rows;
  // one-shot k splits: gw.cnt set, the splits of each tile group are summed inside the launch (the host
  // sets it only when the grid is resident at once); otherwise gemm_os_epilogue_kernel sums them
  GroupWait gw;
  RopeOut ro;                         // EPI_BIAS (qkv) on the register-weight kernel: ro.rope set, see RopeOut
};

// Launch configurations (see gemm.hip); the host picks one per projection.
enum GemmCfg : int { CFG_QKV = 0, CFG_OPROJ = 1, CFG_GATE_UP = 2, CFG_DOWN = 3, CFG_LM_HEAD = 4 };
// tiles_per_wg: the padding unit of the packed tile count (every kernel of the projection divides it)
struct GemmShape { int tiles_per_wg; int waves; };
GemmShape gemm_shape(int cfg);
// The kernel and grid a launch uses.  GK_ONESHOT (M <= 32) and GK_MM (larger M, not the lm_head) pick
// their own k split; GK_STREAM (the lm_head, or shapes the others do not take) runs stream_split.
// Streaming and one-shot launches have groups x ksplit x mchunks workgroups; the large-M kernel
// covers nbm x nbn blocks of config mm_id.  part_floats: split partials.  Sets a.kps.
// GK_MM takes its activations already normalised (the caller runs norm_rows once instead of every
// column block normalising its rows again): a launch with XF_RMS in its configuration must not pass
// GK_MM rows that still need the norm.
enum GemmKind : int { GK_STREAM = 0, GK_ONESHOT = 1, GK_MM = 2 };
struct GemmPlan {
  int kind; int ksplit; int tiles_per_wg; int groups; int mchunks; size_t part_floats;
  int mm_id; int nbm; int nbn;
  int tail_full, tail_split;  // GK_STREAM: see GemmP (set in both)
  int mrows;                  // GK_ONESHOT: rows per m-chunk (blockIdx.z), 32, or 16 for half-row chunks
};
// How large-M launches are planned.  target_wgs / min_stages: k is split only while the launch has fewer
// than target_wgs workgroups, and only into splits of at least min_stages stages.  wr_ops: the
// projections (bit cfg) that may take the register-weight kernel, from wr_min_rows rows (0: from 2048
// rows for gate_up and down, 4096 for qkv and o_proj, 256 for the lm_head, where it measured faster
// than the LDS-staged and streaming kernels).
struct MmPolicy {
  int target_wgs = 256;
  int min_stages = 8;
  int wr_ops = (1 << CFG_QKV) | (1 << CFG_OPROJ) | (1 << CFG_GATE_UP) | (1 << CFG_DOWN) | (1 << CFG_LM_HEAD);
  int wr_min_rows = 0;
  int wr_small_ops = (1 << CFG_QKV) | (1 << CFG_OPROJ);  // take the 64 x 128 register-weight blocks below the 128 x 256 ones
  // gate_up / down below 256 rows: -1 the measured choice of register-weight blocks, else bit 0 / 1 the 64 x 128
  // blocks, bit 2 / 3 the 128 x 128 ones (0: the LDS-staged kernel)
  int wr_ffn = -1;
  int force_split = 0;  // > 1: this k split whenever it divides the stages (the fused o_proj + norm)
  int wr3 = 1;          // o_proj / down at the register-weight thresholds: 128 x 192 blocks (0: 128 x 256)
  int wt8 = 1;  // LDS-staged 128 x 192 blocks of eight waves (bit 0 gate_up, bit 1 down) instead of four
  int wt256 = 512;  // gate_up from 257 up to this many rows on LDS-staged 256 x 192 blocks of eight waves
  // the streaming lm_head of up to 32 rows: the column groups past the last whole round over this many
  // compute units (one group per unit per round) split k up to 3 ways, so that every unit streams about
  // the same bytes (0: off)
  int lm_tail_cus = 0;
  // one-shot projections (bit cfg) of 17 to 32 rows run as two 16-row m-chunks: each workgroup takes in
  // half the activations for the same weight tile
  int os_half = (1 << CFG_QKV) | (1 << CFG_OPROJ);
};
GemmPlan gemm_plan(int cfg, GemmP& a, int stream_split, const MmPolicy& pol = MmPolicy{});
// whether the plan runs the one-shot register-fragment body, the only one that takes xfrag / yfrag 1
bool gemm_takes_frag(int cfg, const GemmPlan& p);
// whether the plan runs the large-M LDS-staged kernel, the only one that takes xfrag 2
bool gemm_takes_blocks(const GemmPlan& p);
// whether the qkv plan's kernel applies RoPE in its epilogue when GemmP::ro is set
bool gemm_ropes_in_epilogue(int cfg, const GemmPlan& p);
hipError_t launch_gemm(int dt, int cfg, const GemmP& a, const GemmPlan& p, hipStream_t st);

// ---- confidence ---------------------------------------------------------------------------------
hipError_t launch_confidence_combine(const float* sm, const int32_t* sa, const float* ss, int tiles, int rows,
                                     int32_t* ids, float* maxp, hipStream_t st);
hipError_t launch_confidence_tiles(const float* logits, int ld, int vocab, int rows, float* sm, int32_t* sa,
                                   float* ss, hipStream_t st);

// ---- the decode loop's threshold unmask (unmask.hip, confidence.hpp) ------------------------------
// Words of an unmask report (int32): the sequence number (written last), masks left in the sub-block,
// rows unmasked, the unshifted argmax of the last confidence row, the block after the update, then the
// sub-block's shifted ids and probabilities (fp32 bits) and the masked / selected row bitmasks (64 bits
// each, as a low and a high word).
constexpr int REP_SEQ = 0, REP_LEFT = 1, REP_COUNT = 2, REP_LAST = 3, REP_BLOCK = 4;
__host__ __device__ constexpr int report_words(int bd, int sub) { return REP_BLOCK + bd + 2 * sub + 4; }

struct UnmaskP {
  int rows;            // confidence rows of the call
  int row0;            // confidence row of block row s0 (s0 for a full step, 0 for a partial one)
  int32_t* block;      // [bd] ids of the active block (device), updated in place
  int bd;              // block length
  int s0, sub;         // the sub-block [s0, s0 + sub); sub = 0: no unmask (an append step)
  int32_t mask_id;
  float thr;           // threshold, rounded to fp32 toward -inf (numpy's fp32 > Python-float decision)
  int32_t* report;     // optional: report_words(bd, sub) words, written when the update is done
  int32_t seq;
};

// Fused confidence combine of the lm_head tile statistics (rows u.rows) + the unmask of u; ids / maxp
// (optional) receive the unshifted confidence as launch_confidence_combine writes it.
hipError_t launch_confidence_unmask(const float* sm, const int32_t* sa, const float* ss, int tiles, int stat_rows,
                                    int32_t* ids, float* maxp, const UnmaskP& u, hipStream_t st);
// The unmask of u on a given confidence ids / maxp [u.rows].
hipError_t launch_unmask(const int32_t* ids, const float* maxp, const UnmaskP& u, hipStream_t st);

// ---- row kernels --------------------------------------------------------------------------------
// k and v (bytes each, 16-byte multiples at 16-byte aligned addresses) copied to kd and vd in one launch
hipError_t launch_kv_copy(const void* k, const void* v, void* kd, void* vd, size_t bytes, hipStream_t st);
hipError_t launch_embed(const int32_t* ids, int n, const uint16_t* table, int vocab, int hidden, uint16_t* out,
                        hipStream_t st);
// copy the input rows into the residual stream and emit their per-16-column sums of squares; hfrag: h
// in MFMA-fragment order (rows <= 32)
hipError_t launch_load_rows(int dt, const uint16_t* x, int rows, int hidden, uint16_t* h, float* ssq, int ssq_ld,
                            hipStream_t st, int hfrag = 0);
// RoPE (cos, sin) table: row r sits at position pos_offset[r / rows_per_seq] + r % rows_per_seq
hipError_t launch_rope_table(int dt, const int32_t* pos_offset, int rows, int rows_per_seq, float neg_log_theta,
                             float* tab, hipStream_t st);
// y = RMSNorm(h) from the sums of squares the producer left (final norm); hfrag: h in MFMA-fragment order;
// yblk: y in the large-M kernel's fragment blocks (frag_blk_off) instead of row-major
hipError_t launch_norm_rows(int dt, const uint16_t* h, int rows, int hidden, const float* ssq, int ssq_ld,
                            const uint16_t* w, float eps, uint16_t* y, hipStream_t st, int hfrag = 0, int yblk = 0);
// The k-split sum of an EPI_RESID projection (row-major partials of part_rows launches) with its residual
// epilogue (h updated in place, per-tile sums of squares to ssq, the exact arithmetic of the split-sum
// kernel), then the next RMSNorm of the new rows (norm_rows_kernel's arithmetic) into y (yblk: fragment
// blocks), in one launch.
hipError_t launch_resid_norm(int dt, const float* part, int splits, int rows, int hidden, uint16_t* h, float* ssq,
                             int ssq_ld, const uint16_t* w, float eps, uint16_t* y, int yblk, hipStream_t st);

// ---- attention ----------------------------------------------------------------------------------
constexpr int MAX_SEQ_UNITS = 128;      // attn_seq_kernel work units (key splits of the sequences)
constexpr int SEQ_CNT_MAX = 16384;      // its arrival counters (sequence, kv head, query tile)
struct AttnP {
  const uint16_t* qkv; int ldq;       // [rows][ldq]: q | k | v, bias added, before RoPE
  int rows, nq, nkv;
  const float* rope;                  // [rows][64][2] RoPE (cos, sin) of row r (position pos_offset + r), model-dtype values;
                                      // null (chunk and loop kernels): the queries arrive rotated and ws >= Lk (no rows taken
                                      // from qkv or appended)
  uint16_t* kc; uint16_t* vc;         // this layer's cache [cap][nkv][128]
  int ws;                             // rows [ws, ws + rows) are this call's: taken from qkv, written to the cache
  int Lk;                             // attended keys [0, Lk)
  float scale;
  int mask;                           // 0 none, 1 block-causal, 2 additive bias
  int q_pos0; int block;              // block-causal: query row r sits at q_pos0 + r
  const float* bias; long long bias_ld;
  int S, chunk;                       // key splits (gridDim.z), keys per split (multiple of 32)
  int target_wgs;                     // workgroups the plan aims for (attn_plan)
  int prefill_hpw;                    // query heads per workgroup of the prefill kernel (0: chosen per launch)
  int prefill_pair;                   // paired-query-block prefill kernel: 0 off, 1 by size, 2 always all heads per
                                      // workgroup, 3 always the heads split over workgroups
  int seq_attn;                       // batched calls without a mask: attn_seq_kernel (no key splits) instead of chunks + merge
  float* part;                        // split partials (merged by attn_merge_kernel)
  uint16_t* out;                      // [rows][nq * 128]
  int ofrag;                          // out in MFMA-fragment order (frag_off; rows <= 32, nseq 1)
  // batched call (nseq > 1, chunked kernel only): sequence b owns rows [b rows, (b + 1) rows) of qkv,
  // rope and out, the cache at kc / vc + b seq_stride, writes from seq_ws[b] and attends
  // [0, seq_lk[b]); ws and Lk above then hold the largest window (S and chunk are planned for it)
  int nseq; long long seq_stride;
  int seq_ws[MAX_SEQS]; int seq_lk[MAX_SEQS];
  // attn_seq_kernel's work units (plan_seq_units), in launch order: a unit is split j of the s splits of
  // sequence b's 64-key blocks, blocks [tb, te), whose partials sit at index u0 + j (a sequence's splits
  // take consecutive indices from u0).  unit_a = b | j << 6 | s << 11 | u0 << 16, unit_t = tb | te << 16.
  // Splits of one sequence leave fp32 partials in part; the last of them to arrive (seq_cnt, zero between
  // launches) merges them in split order.
  int nunits;
  unsigned* seq_cnt;
  int unit_a[MAX_SEQ_UNITS]; int unit_t[MAX_SEQ_UNITS];
  // the qkv epilogue has already RoPE'd the queries into out and appended the K/V rows (GemmP::ro): the
  // launch skips rope_kv_kernel
  int roped;
};
struct AttnPlan { int chunked; int q_tiles_per_wg; int key_groups; int qg; int S; int chunk; };
AttnPlan attn_plan(int rows, int nq, int nkv, int Lk, int target_wgs, int nseq);
// whether launch_attention starts with rope_kv_kernel for a (the batched-sequence and prefill kernels)
bool attn_takes_roped(const AttnP& a);
// attn_seq_kernel's units for a batched call (a.nseq, rows, heads, seq_lk and seq_cnt set): each sequence
// starts as one unit; while fewer than ncu / (nkv x query-tile groups) units exist (one workgroup per
// compute unit), the sequence with the longest split (lowest index on ties) takes one more split, until
// the longest split is at most 2 blocks.  ncu 0 or no counters: no splits.  Returns the partial floats
// the splits need (0 without splits).
size_t plan_seq_units(AttnP& a, int ncu);
hipError_t launch_attention(int dt, const AttnP& a, hipStream_t st);
size_t attn_partial_floats(const AttnP& a);


}  // namespace fdllm
