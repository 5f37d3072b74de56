/* CPU restatement of the per-row confidence and the threshold unmask rule.  TEST INFRASTRUCTURE ONLY.
 *
 * Follows the reference:
 *   shifted_confidence   fast_dllm_relax/runtime.py:158-181 (argmax first index; max softmax prob)
 *   device confidence    fast_dllm_relax/model/metal.py:316-374 (maxp = 1 / sum_j exp(x_j - max))
 *   unmask rule          fast_dllm_relax/runtime.py:794-805 (rows with p > threshold among the masked
 *                        rows, else the first masked row of maximal p)
 *
 * The confidence is defined with a fixed evaluation order so that the HIP kernels and this file give
 * identical bits for identical logits:
 *   - e(x), x <= 0: Cody-Waite reduction x = n ln2 + r (ln2 split in a 16-bit head and a tail), a
 *     degree-7 Taylor polynomial of exp(r) in Horner form with fused multiply-adds, then r scaled by
 *     2^n built in the exponent field; e(x) = 0 for x < -86 (no subnormals).  Every step is an IEEE
 *     fp32 operation, so a C compiler with -ffp-contract=off and the HIP compiler with contraction
 *     off evaluate it identically.
 *   - a row of V logits is cut into tiles of 256 (tile t covers [256t, 256t+256)).  For each tile:
 *     m_t = max, a_t = first index attaining m_t, and s_t = sum of e(x - m_t) evaluated as 64 lane
 *     partials (lane l adds j = 256t + l + 64i, i = 0..3, in increasing i, skipping j >= V), then a
 *     butterfly over the lanes: for k = 32,16,8,4,2,1: v[l] = v[l] + v[l ^ k].
 *   - row: M = max_t m_t; argmax = a_t of the first tile with m_t == M; S = lane partials
 *     (lane l adds s_t * e(m_t - M) for t = l, l+64, ... in increasing t; product rounded, then the
 *     add rounded), then the same butterfly; maxp = 1 / S.
 * In real arithmetic S = sum_j exp(x_j - M), so maxp is the reference's max softmax probability.
 *
 * Pinned by tests/test_oracle_pinning.py: e(x) against float64 exp (<= 2 ulp over [-86, 0]), maxp
 * against a float64 softmax (relative 1e-6), argmax against numpy's first-index argmax, and the unmask
 * rule against a brute-force restatement of runtime.py:794-805 on random small cases.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define FD_TILE 256
#define FD_LANES 64

static float fd_bits_to_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float fd_exp_neg(float x) {
    if (x != x) return x;
    if (x < -86.0f) return 0.0f;
    const float log2e = 1.44269502162933349609375f;   /* 0x3FB8AA3B */
    const float ln2_hi = 0.693145751953125f;           /* 0x3F317200 */
    const float ln2_lo = 1.428606765330187045e-06f;    /* 0x35BFBE8E */
    float n = rintf(x * log2e);
    float r = fmaf(n, -ln2_hi, x);
    r = fmaf(n, -ln2_lo, r);
    float p = 1.98412701e-4f;                          /* 1/5040 */
    p = fmaf(p, r, 1.38888892e-3f);                    /* 1/720 */
    p = fmaf(p, r, 8.33333377e-3f);                    /* 1/120 */
    p = fmaf(p, r, 4.16666679e-2f);                    /* 1/24 */
    p = fmaf(p, r, 1.66666672e-1f);                    /* 1/6 */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int ni = (int)n;
    float scale = fd_bits_to_float((uint32_t)(ni + 127) << 23);
    return p * scale;
}

static void butterfly(float* v) {
    float t[FD_LANES];
    for (int k = 32; k >= 1; k >>= 1) {
        for (int l = 0; l < FD_LANES; ++l) t[l] = v[l] + v[l ^ k];
        memcpy(v, t, sizeof(t));
    }
}

/* Per-tile statistics of one row: m[t], a[t], s[t] for t < ceil(V/256). */
void fd_tile_stats(const float* x, int vocab, float* m, int32_t* a, float* s) {
    int tiles = (vocab + FD_TILE - 1) / FD_TILE;
    for (int t = 0; t < tiles; ++t) {
        int j0 = t * FD_TILE, j1 = j0 + FD_TILE < vocab ? j0 + FD_TILE : vocab;
        float mx = x[j0];
        int32_t am = j0;
        for (int j = j0 + 1; j < j1; ++j) {
            if (x[j] > mx) { mx = x[j]; am = j; }
        }
        float v[FD_LANES];
        for (int l = 0; l < FD_LANES; ++l) {
            float acc = 0.0f;
            for (int i = 0; i < FD_TILE / FD_LANES; ++i) {
                int j = j0 + l + FD_LANES * i;
                if (j < j1) acc = acc + fd_exp_neg(x[j] - mx);
            }
            v[l] = acc;
        }
        butterfly(v);
        m[t] = mx; a[t] = am; s[t] = v[0];
    }
}

/* Combine of the tile statistics of one row into (argmax, maxp). */
void fd_combine(const float* m, const int32_t* a, const float* s, int tiles, int32_t* id, float* maxp) {
    float mx = m[0];
    int32_t am = a[0];
    for (int t = 1; t < tiles; ++t) {
        if (m[t] > mx) { mx = m[t]; am = a[t]; }
    }
    float v[FD_LANES];
    for (int l = 0; l < FD_LANES; ++l) {
        float acc = 0.0f;
        for (int t = l; t < tiles; t += FD_LANES) {
            float w = s[t] * fd_exp_neg(m[t] - mx);
            acc = acc + w;
        }
        v[l] = acc;
    }
    butterfly(v);
    *id = am;
    *maxp = 1.0f / v[0];
}

/* Unshifted confidence of rows x [rows, vocab] -> ids [rows], maxp [rows]. */
void fd_confidence(const float* logits, int rows, int vocab, int32_t* ids, float* maxp,
                   float* m_tmp, int32_t* a_tmp, float* s_tmp) {
    int tiles = (vocab + FD_TILE - 1) / FD_TILE;
    for (int r = 0; r < rows; ++r) {
        fd_tile_stats(logits + (size_t)r * vocab, vocab, m_tmp, a_tmp, s_tmp);
        fd_combine(m_tmp, a_tmp, s_tmp, tiles, ids + r, maxp + r);
    }
}

/* Threshold unmask (runtime.py:794-805): masked[r] != 0 marks a mask position among n rows.
 * Writes sel[r] = 1 for the rows to unmask; returns how many were selected (0 when no row is masked).
 * thr is the float32 rounding toward -inf of the host threshold, which makes `p > thr` the same
 * decision as numpy's float32-vs-Python-float comparison. */
int fd_unmask(const float* p, const uint8_t* masked, int n, float thr, uint8_t* sel) {
    int count = 0, best = -1;
    float bestp = 0.0f;
    for (int r = 0; r < n; ++r) {
        sel[r] = 0;
        if (!masked[r]) continue;
        if (p[r] > thr) { sel[r] = 1; ++count; }
        if (best < 0 || p[r] > bestp) { best = r; bestp = p[r]; }
    }
    if (count == 0 && best >= 0) { sel[best] = 1; count = 1; }
    return count;
}
