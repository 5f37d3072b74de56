/* C ABI of the MI355X-native cached block-diffusion step (libfdllm.so).
 *
 * Replaces the reference's TVM Relax VM function table for Fast-dLLM v2: the artifact exposes
 * REQUIRED_FNS (fast_dllm_relax/export_utils.py:13-17), called as vm["name"](..., params) by
 * fast_dllm_relax/runtime.py.  Every entry point below keeps the argument meaning, shapes and error
 * behaviour of the reference function it names; shapes are passed as plain ints and tensors as device
 * pointers (the caller owns every buffer; the KV caches are mutated in place, as in the reference).
 *
 * Conventions
 *   - All pointers are device pointers unless stated; `stream` is a hipStream_t (NULL = default).
 *   - Activations/weights/caches are in the context's dtype (bf16 or fp16, 2-byte elements);
 *     logits are fp32; token ids are int32.  Weights, activations, caches and logits must be
 *     16-byte aligned (FDLLM_EINVAL otherwise); id, offset and bias arrays need only their
 *     element alignment.
 *   - KV caches: [num_layers, 1, cap, num_kv_heads, head_dim] rows (contract "inplace_bsnh_v1",
 *     export_utils.py:21-34).
 *   - Return value: 0 on success; FDLLM_EINVAL for a rejected argument (the reference raises
 *     ValueError / a VM shape error); FDLLM_EHIP for a HIP runtime failure; FDLLM_ESTATE when weights
 *     are not bound.  fdllm_last_error() returns this thread's message for the last failure.
 *   - All work is enqueued on `stream`; nothing synchronises the host unless stated.  One context
 *     per stream; a context is not thread-safe.
 */
#ifndef FDLLM_H
#define FDLLM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FDLLM_OK 0
#define FDLLM_EINVAL 1
#define FDLLM_EHIP 2
#define FDLLM_ESTATE 3

#define FDLLM_DTYPE_BF16 0
#define FDLLM_DTYPE_F16 1

typedef struct fdllm_ctx fdllm_ctx;

/* Model constants; mirror of FastDLLMRelaxConfig (fast_dllm_relax/model/cuda.py:15-29). */
typedef struct fdllm_config {
  int32_t vocab_size;
  int32_t hidden_size;
  int32_t intermediate_size;
  int32_t num_hidden_layers;
  int32_t num_attention_heads;
  int32_t num_key_value_heads;
  int32_t head_dim;            /* 128 for the HIP attention kernel */
  float rms_norm_eps;
  float rope_theta;
  int32_t tie_word_embeddings;
  int32_t bd_size;             /* block size (32); partial steps use bd_size / 4 rows */
  int32_t dtype;               /* FDLLM_DTYPE_* */
  int32_t max_rows;            /* rows the workspace is sized for at creation (grown on demand) */
} fdllm_config;

/* Replaces tvm.relax.VirtualMachine(load_module(...)) (fast_dllm_relax/runners.py:614-615). */
int fdllm_create(const fdllm_config* cfg, fdllm_ctx** out);
void fdllm_destroy(fdllm_ctx* ctx);

/* Number of packed parameters and their names, in param_names.txt order
 * (fast_dllm_relax/runners.py:947-972; 198 for the tied 1.5B model). */
int fdllm_num_params(const fdllm_ctx* ctx);
const char* fdllm_param_name(const fdllm_ctx* ctx, int index);

/* Binds the packed `params` list (cuda.py:807, "param_mode": "packed"): n device pointers in
 * fdllm_param_name order, each 16-byte aligned (FDLLM_EINVAL otherwise).  The caller keeps them alive
 * while the context uses them. */
int fdllm_bind_weights(fdllm_ctx* ctx, const void* const* ptrs, int n);

/* embed (cuda.py:698-699): ids [seq_len] int32 -> out [seq_len, hidden]. */
int fdllm_embed(fdllm_ctx* ctx, const int32_t* ids, int seq_len, void* out, void* stream);

/* forward_hidden (cuda.py:604-608, 701-702): stateless forward of [1, seq_len, hidden] with the
 * additive attention bias [1, 1, seq_len, seq_len] fp32; bias == NULL means the block-causal bias of
 * build_prefix_block_attention_bias(0, seq_len, block_size=bd_size) (cuda.py:148-177). */
int fdllm_forward_hidden(fdllm_ctx* ctx, const void* input_embed, int seq_len, const float* attention_bias,
                         void* out, void* stream);

/* get_logits (cuda.py:704-711): hidden [rows, hidden] -> logits [rows, vocab] fp32 (rounded to the
 * model dtype first, as the reference's model-dtype GEMM output is). */
int fdllm_get_logits(fdllm_ctx* ctx, const void* hidden, int rows, float* logits, void* stream);

/* build_prefix_cache (cuda.py:610-637, 713-721): writes rows [0, prefix_len) of every layer of the
 * caches in place; prefix_bias as in fdllm_forward_hidden (NULL = block-causal). */
int fdllm_build_prefix_cache(fdllm_ctx* ctx, const void* prefix_embed, int prefix_len, const float* prefix_bias,
                             void* k_cache, void* v_cache, int cap, void* stream);

/* forward_cached (cuda.py:723-738, 639-666 with fast_dllm.attn_inplace, runtime.py:63-73): writes the
 * block's K/V at rows [prefix_len, prefix_len + block_len) and attends over [0, prefix_len + block_len).
 * cache_offset: device int32 scalar, RoPE position of row 0.  out [block_len, hidden]. */
int fdllm_forward_cached(fdllm_ctx* ctx, const void* active_embed, int block_len, void* k_cache, void* v_cache,
                         int cap, const int32_t* cache_offset, int64_t prefix_len, void* out, void* stream);

/* Allocation-free variant of fdllm_forward_cached.  It has no counterpart in the reference: it is for
 * callers that cannot allocate device memory inside a call (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, semantics and results (bit for bit) as
 * fdllm_forward_cached, but the step's workspace (residual stream, projections, norms, RoPE table and
 * the split partials of the projections and the attention) lives in a fixed 24 MiB device array of the
 * library, one per GPU, held until the process ends, and the call allocates and frees nothing.
 * Limits: at most 32 rows, and the attended keys must fit the scratch (the 1.5B shapes: up to 8192
 * keys through the chunked attention, more through the looped one); larger calls return FDLLM_EINVAL.
 * Every call on one GPU shares that GPU's array and leaves its contents behind: calls that overlap on
 * one GPU (two streams, threads or contexts) race. */
int fdllm_forward_cached_noalloc(fdllm_ctx* ctx, const void* active_embed, int block_len, void* k_cache,
                                 void* v_cache, int cap, const int32_t* cache_offset, int64_t prefix_len, void* out,
                                 void* stream);

/* forward_block_partial_rp{0,8,16,24} (cuda.py:740-788): bd_size/4 rows written at
 * [prefix_len + rp, + bd_size/4), attending over [0, prefix_len + bd_size). */
int fdllm_forward_block_partial(fdllm_ctx* ctx, int replace_position, const void* active_embed, int rows,
                                void* k_cache, void* v_cache, int cap, const int32_t* cache_offset,
                                int64_t prefix_len, void* out, void* stream);
int fdllm_forward_block_partial_rp0(fdllm_ctx* ctx, const void* active_embed, int rows, void* k_cache,
                                    void* v_cache, int cap, const int32_t* cache_offset, int64_t prefix_len,
                                    void* out, void* stream);
int fdllm_forward_block_partial_rp8(fdllm_ctx* ctx, const void* active_embed, int rows, void* k_cache,
                                    void* v_cache, int cap, const int32_t* cache_offset, int64_t prefix_len,
                                    void* out, void* stream);
int fdllm_forward_block_partial_rp16(fdllm_ctx* ctx, const void* active_embed, int rows, void* k_cache,
                                     void* v_cache, int cap, const int32_t* cache_offset, int64_t prefix_len,
                                     void* out, void* stream);
int fdllm_forward_block_partial_rp24(fdllm_ctx* ctx, const void* active_embed, int rows, void* k_cache,
                                     void* v_cache, int cap, const int32_t* cache_offset, int64_t prefix_len,
                                     void* out, void* stream);

/* The reference's attention callbacks, for a model that computes its own projections and RoPE and calls
 * out once per layer for the cache write and the attention (fast_dllm_relax/runtime.py:19-80, called
 * from model/cuda.py through rx.call_inplace_packed).  Tensors are BSNH with batch 1, in the context's
 * dtype: k / v [rows, nkv, head_dim], q / out [rows, nq, head_dim]; the caches [L, 1, cap, nkv,
 * head_dim] are the ones the other entry points take.  Neither call needs bound weights.
 *
 * fast_dllm.kv_write (runtime.py:76-80, _write_rows :51-60): k / v copied byte for byte to cache rows
 * [start, start + rows) of `layer`.  FDLLM_EINVAL: "KV write [s, e) outside cache capacity cap". */
int fdllm_kv_write(fdllm_ctx* ctx, const void* k, const void* v, int rows, void* k_cache, void* v_cache, int cap,
                   int layer, int64_t start, void* stream);

/* fast_dllm.attn_inplace (runtime.py:63-73): the write of fdllm_kv_write at rows [prefix_len + write_rel,
 * + rows), then out = softmax(q K^T / sqrt(head_dim)) V over cache rows [0, prefix_len + attend_rel) of
 * `layer`, no mask, query head h on kv head h / (nq / nkv) (_attend, runtime.py:30-48); like the
 * reference's slice of the cache, the attended rows stop at the capacity.  q must already be rotated.
 * FDLLM_EINVAL: "KV write [s, e) past the attended rows [0, n)" when the written rows end past the
 * attended ones, and the capacity error of fdllm_kv_write.  q, the caches and out must be 16-byte
 * aligned. */
int fdllm_attn_inplace(fdllm_ctx* ctx, const void* q, const void* k, const void* v, int rows, void* k_cache,
                       void* v_cache, int cap, int layer, int64_t prefix_len, int write_rel, int attend_rel,
                       void* out, void* stream);

/* Batched steps: no counterpart in the reference, whose entry points are batch 1
 * (fast_dllm_relax/model/cuda.py:796-836); they serve callers that refine one block per sequence
 * for many sequences at once.  nseq (<= 64) sequences share one cache tensor [L, nseq, cap, nkv, hd]
 * (inplace_bsnh_v1, export_utils.py:21-34, with a batch dimension); active_embed is [nseq, rows, H]
 * and out the same shape.  cache_offset is a device int32 [nseq] (row 0's RoPE position per
 * sequence) and prefix_lens a host int64 [nseq].  Each sequence follows the batch-1 semantics
 * exactly: fdllm_forward_cached_batch writes rows [P_b, P_b + rows) and attends [0, P_b + rows);
 * fdllm_forward_block_partial_batch writes [P_b + rp, + bd_size/4) and attends [0, P_b + bd_size).
 * Window errors name the sequence. */
int fdllm_forward_cached_batch(fdllm_ctx* ctx, const void* active_embed, int nseq, int rows, void* k_cache,
                               void* v_cache, int cap, const int32_t* cache_offset, const int64_t* prefix_lens,
                               void* out, void* stream);
int fdllm_forward_block_partial_batch(fdllm_ctx* ctx, int replace_position, const void* active_embed, int nseq,
                                      int rows, void* k_cache, void* v_cache, int cap, const int32_t* cache_offset,
                                      const int64_t* prefix_lens, void* out, void* stream);
/* build_prefix_cache (cuda.py:610-637) of sequence `seq` into its slice of a batched cache
 * [L, nseq, cap, nkv, hd]; the other sequences' rows are untouched. */
int fdllm_build_prefix_cache_seq(fdllm_ctx* ctx, const void* prefix_embed, int prefix_len, const float* prefix_bias,
                                 void* k_cache, void* v_cache, int cap, int nseq, int seq, void* stream);

/* Fused lm_head + confidence: the device restatement of get_confidence_m{rows}
 * (fast_dllm_relax/model/metal.py:505-528, dispatch runtime.py:136-174).  ids [rows] int32 = first
 * argmax of each row's logits; maxp [rows] fp32 = 1 / sum exp(logit - max).  Unshifted; the caller
 * applies the shift of runtime.py:172-174.  logits may be NULL, or [rows, vocab] fp32 to also receive
 * exactly what fdllm_get_logits returns. */
int fdllm_get_confidence(fdllm_ctx* ctx, const void* hidden, int rows, int32_t* ids, float* maxp, float* logits,
                         void* stream);

/* The same confidence of given fp32 logits [rows, ld] (the host reduction of runtime.py:176-181). */
int fdllm_confidence_from_logits(fdllm_ctx* ctx, const float* logits, int rows, int vocab, int ld, int32_t* ids,
                                 float* maxp, void* stream);

/* Threshold unmask of one sub-block on the device: the rule of fast_dllm_relax/runtime.py:794-805 (the
 * masked rows whose max probability is above `threshold`, else the first masked row of largest
 * probability) with the shift of runtime.py:172-174, replacing the host loop's per-step readback of the
 * confidence (runtime.py:179-181; device-confidence precedent model/metal.py:316-374).
 *   ids, maxp   [rows] unshifted confidence of one model call, as fdllm_get_confidence writes it.
 *   block       [bd_size] int32 ids of the active block (device); block rows [s0, s0 + sub_rows) are the
 *               sub-block, and block row s0 + r reads the shifted confidence row row0 + r (that is, the
 *               prediction of row row0 + r - 1; row 0 its own): row0 = s0 for a full 32-row step,
 *               0 for a partial step.  The selected rows are overwritten with their predicted ids.
 *   threshold   compared as `p > threshold` in fp32 (pass the fp32 rounding toward -inf of the host
 *               threshold to reproduce numpy's fp32-vs-Python-float comparison).
 *   report      optional int32 [4 + bd_size + 2 sub_rows + 4] (device memory, or host memory from
 *               fdllm_host_alloc that the host polls): word 0 = seq, written after everything else;
 *               1 = masked rows left in the sub-block; 2 = rows unmasked; 3 = unshifted argmax of the
 *               last confidence row (the append step's next token, runtime.py:360-363); 4.. = the block
 *               after the update; then the sub-block's shifted ids, their probabilities (fp32 bits), and
 *               the 64-bit masks of the rows that were masked and that were selected, each as a low and
 *               a high word (bit r: sub-block row r).
 * sub_rows = 0 updates nothing (an append step that only needs the report).  bd_size must be <= 64. */
int fdllm_unmask(fdllm_ctx* ctx, const int32_t* ids, const float* maxp, int rows, int row0, int32_t* block, int s0,
                 int sub_rows, int32_t mask_id, float threshold, int32_t* report, int32_t seq, void* stream);

/* The fused north-star head of one decode step: lm_head + max-softmax / first-argmax over the vocabulary
 * (fdllm_get_confidence) + the threshold unmask of fdllm_unmask, in two launches and without a
 * readback.  ids / maxp: optional (both or neither) [rows] outputs of the unshifted confidence. */
int fdllm_get_confidence_unmask(fdllm_ctx* ctx, const void* hidden, int rows, int row0, int32_t* block, int s0,
                                int sub_rows, int32_t mask_id, float threshold, int32_t* ids, float* maxp,
                                int32_t* report, int32_t seq, void* stream);

/* Pinned, device-mapped, coherent host memory for unmask reports (zeroed): the host polls what the
 * device writes there instead of waiting for a copy.  No reference counterpart (the reference reads
 * the confidence back with a blocking copy, runtime.py:179-181). */
int fdllm_host_alloc(size_t bytes, void** host_ptr, void** device_ptr);
void fdllm_host_free(void* host_ptr);

/* Profiling hook; it has no counterpart in the reference.  Launches one operator of the cached step
 * `iters` times back to back on `stream`, reading and writing the context's own workspace (the values
 * are not meaningful); launch i uses layer (layer + i) % num_layers, as a step walks the layers, so a
 * benchmark can time one kernel with events on the stream it runs on without re-reading one layer's
 * weights from cache.  FDLLM_OP_ATTENTION attends rows [0, attend_len) of each layer of the caches. */
#define FDLLM_OP_QKV 0
#define FDLLM_OP_O_PROJ 1
#define FDLLM_OP_GATE_UP 2
#define FDLLM_OP_DOWN 3
#define FDLLM_OP_ATTENTION 4
#define FDLLM_OP_LM_HEAD_CONFIDENCE 5
int fdllm_bench_op(fdllm_ctx* ctx, int op, int rows, int layer, int iters, void* k_cache, void* v_cache, int cap,
                   int attend_len, void* stream);

/* Diagnostic; it has no counterpart in the reference.  Number of launches this context has run that
 * reduced their own splits (the down projection's k splits, the decode attention's key splits) instead of
 * handing them to a separate split-sum or merge launch.  Such a launch is planned when its whole grid is
 * resident at once (at most one workgroup per compute unit); FDLLM_GROUP_WAITS=0 at fdllm_create turns
 * it off, and so does a timed-out wait (reported by the next entry point as FDLLM_EHIP). */
long long fdllm_group_wait_launches(const fdllm_ctx* ctx);

/* Diagnostic; it has no counterpart in the reference.  Number of layer-loop calls (cached steps, short
 * stateless forwards) this context has run with the activations in MFMA-fragment order: calls of at
 * most 32 rows whose four projections all take the one-shot GEMM, unless FDLLM_XFRAG=0 was set when
 * the context was created.  Results are the same bit for bit either way. */
long long fdllm_frag_calls(const fdllm_ctx* ctx);

/* Message of this thread's last failure ("" if none). */
const char* fdllm_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* FDLLM_H */
