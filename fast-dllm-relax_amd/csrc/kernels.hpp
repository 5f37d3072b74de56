// Kernel launch interfaces shared by the C ABI (capi.hip) and the kernel files.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fdllm {

enum Epilogue : int { EPI_STORE = 0, EPI_BIAS = 1, EPI_RESID = 2, EPI_SILU = 3, EPI_LOGITS = 4 };

struct GemmArgs {
  const uint16_t* X; int ldx; int M;  // activations [M][ldx]
  const uint16_t* W; int N; int K;    // weights [N][K] (nn.Linear layout)
  int kc;                             // k elements per split (multiple of 128)
  int wg_rows;                        // weight rows advanced per workgroup along blockIdx.x
  int tile_stride;                    // row distance between the tiles of one wave
  float* partial;                     // split-K partials
  int* counters;                      // split-K arrival counters (zero between launches)
  uint16_t* Y; int ldy;               // output
  const uint16_t* bias;               // EPI_BIAS
  const uint16_t* resid; int ldr;     // EPI_RESID (may alias Y)
  float* logits; int ldl;             // EPI_LOGITS (optional)
  float* stat_m; int32_t* stat_a; float* stat_s; int stat_tiles;  // EPI_LOGITS confidence tiles
};

hipError_t launch_gemm(int dt, int epi, int tpw, int mt, const GemmArgs& a, int nblocks, int ksplit, int mchunks,
                       hipStream_t st);
hipError_t launch_confidence_combine(const float* sm, const int32_t* sa, const float* ss, int tiles, int rows,
                                     int32_t* ids, float* maxp, hipStream_t st);
hipError_t launch_confidence_tiles(const float* logits, int ld, int vocab, int rows, float* sm, int32_t* sa,
                                   float* ss, hipStream_t st);

hipError_t launch_embed(const int32_t* ids, int n, const uint16_t* table, int vocab, int hidden, uint16_t* out,
                        hipStream_t st);
hipError_t launch_rmsnorm(int dt, const uint16_t* x, int ldx, int rows, int hidden, const uint16_t* w, float eps,
                          uint16_t* y, int ldy, hipStream_t st);

struct RopeArgs {
  const uint16_t* qkv; int ld;       // [R][ld]: q | k | v, pre-RoPE, bias added
  int rows, nq, nkv, hd;
  const int32_t* pos_offset;         // device int32: absolute position of row 0
  float neg_log_theta;               // (float)(-ln(theta))
  uint16_t* q_out;                   // [R][nq * hd]
  uint16_t* k_cache; uint16_t* v_cache;  // this layer's [cap][nkv][hd]
  int write_start;                   // first cache row written
};
hipError_t launch_rope_kv(int dt, const RopeArgs& a, hipStream_t st);

struct AttnArgs {
  const uint16_t* q;                 // [R][nq * hd] rotated queries
  const uint16_t* k; const uint16_t* v;  // this layer's cache [>= Lk][nkv][hd]
  int rows, nq, nkv, hd;
  int Lk;                            // attended rows [0, Lk)
  float scale;
  int mask;                          // 0 none, 1 block-causal, 2 additive bias
  int q_pos0;                        // absolute position of query row 0 (block-causal)
  int block;                         // block size (block-causal)
  const float* bias; long long bias_ld;  // bias[r * ld + key] (mask 2)
  int nsplit, chunk;                 // key splits (gridDim.z) and keys per split (multiple of 64)
  float* o_part; float* m_part; float* l_part;  // [nsplit][nkv][QRp][hd], [nsplit][nkv][QRp]
  int QRp;                           // padded rows per kv head (multiple of 16)
  uint16_t* out;                     // [R][nq * hd]
};
hipError_t launch_attention(int dt, const AttnArgs& a, int nqgroups, hipStream_t st);

}  // namespace fdllm
