/*
 * CPU oracle for the decoder-layer operators around the packed matmul:
 * rmsnorm, rope, kv-write, attention, silu-mul and add.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Each function restates the
 * reference's Rust operator in plain C, in the same evaluation order, and
 * cites the file:line it follows (paths relative to the reference repo
 * root). Rust's f32 `powf`, `exp` and `sin_cos` are the platform libm's
 * powf, expf and sinf/cosf; iterator `sum` is a left fold from zero.
 * Built with -ffp-contract=off (no fused multiply-adds).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "oracle.h"

/* rmsnorm (src/lib.rs:348-402): per row, mean_square = sum(v * v) / cols in
 * f32, scale = 1 / sqrt(mean_square + epsilon), out = v * scale * w. The
 * weight is one row broadcast over every row (w_rows 1) or one row per
 * input row (w_rows == rows). */
int or_rmsnorm(const float *x, uint64_t rows, uint64_t cols, const float *w, uint64_t w_rows, float epsilon,
               float *out) {
  /* the reference rejects epsilon <= 0 only: a NaN epsilon gives NaN rows */
  if (cols == 0 || epsilon <= 0.0f || (w_rows != 1 && w_rows != rows)) return -1;
  for (uint64_t r = 0; r < rows; ++r) {
    const float *v = x + r * cols;
    const float *wv = w + (w_rows == 1 ? 0 : r * cols);
    float sum = 0.0f;
    for (uint64_t c = 0; c < cols; ++c) sum += v[c] * v[c];
    const float mean_square = sum / (float)cols;
    const float scale = 1.0f / sqrtf(mean_square + epsilon);
    for (uint64_t c = 0; c < cols; ++c) out[r * cols + c] = v[c] * scale * wv[c];
  }
  return 0;
}

/* rope (src/lib.rs:427-447, 616-687), unscaled frequencies, all pairs
 * rotated: row r's position is (offset + r) * scale in f32; pair p's
 * frequency base^(-2p / dimension); interleaved pairs (2p, 2p + 1) or
 * half-split pairs (p, p + dimension / 2) inside each of head_count
 * blocks of cols / head_count columns; columns past `dimension` in a block
 * are copied unchanged. */
int or_rope(const float *x, uint64_t rows, uint64_t cols, float base, float scale, uint64_t dimension,
            uint64_t position_offset, uint64_t head_count, int half_split, float *out) {
  if (head_count == 0 || cols % head_count) return -1;
  const uint64_t head_width = cols / head_count;
  if (dimension == 0 || dimension % 2 || dimension > head_width) return -1;
  if (!(base > 0.0f) || !isfinite(base) || !(scale > 0.0f) || !isfinite(scale)) return -1;
  memcpy(out, x, rows * cols * sizeof(float));
  const uint64_t half = dimension / 2;
  for (uint64_t r = 0; r < rows; ++r) {
    const float position = (float)(position_offset + r) * scale;
    for (uint64_t h = 0; h < head_count; ++h) {
      const uint64_t col_base = r * cols + h * head_width;
      for (uint64_t p = 0; p < half; ++p) {
        const float frequency = powf(base, -2.0f * (float)p / (float)dimension);
        const float angle = position * frequency;
        const float s = sinf(angle), c = cosf(angle);
        const uint64_t first = half_split ? col_base + p : col_base + 2 * p;
        const uint64_t second = half_split ? col_base + p + half : col_base + 2 * p + 1;
        const float a = x[first], b = x[second];
        out[first] = a * c - b * s;
        out[second] = a * s + b * c;
      }
    }
  }
  return 0;
}

/* kv-write (src/lib.rs:740-768): rows over the store's rows
 * row_offset .. row_offset + count, in place. */
int or_kv_write(float *store, uint64_t capacity, uint64_t width, const float *rows, uint64_t count,
                uint64_t row_offset) {
  if (row_offset + count > capacity || row_offset + count < row_offset) return -1;
  memcpy(store + row_offset * width, rows, count * width * sizeof(float));
  return 0;
}

/* attention (src/lib.rs:780-990) without window, latent or value-width
 * forms: q [seq, heads * head_dim], k and v [kv_seq, kv_heads * head_dim]
 * (the first key_count rows of the store); the queries are the last `seq`
 * positions; causal masking admits keys up to the query's position. Per
 * (head, query): scores = dot(q, k) * scale in key order, max, exp(s - max),
 * sum, out[d] = sum_j (w_j / sum) * v[j][d] in key order. score_scale NaN
 * means 1 / sqrt(head_dim). */
int or_attention(const float *q, uint64_t seq, const float *k, const float *v, uint64_t kv_seq, uint64_t heads,
                 uint64_t head_dim, uint64_t kv_heads, int causal, float score_scale, float *scores,
                 float *out) {
  if (heads == 0 || head_dim == 0 || kv_heads == 0 || heads % kv_heads || seq > kv_seq) return -1;
  const uint64_t group = heads / kv_heads;
  const uint64_t q_dim = heads * head_dim, kv_dim = kv_heads * head_dim;
  const float scale = isnan(score_scale) ? 1.0f / sqrtf((float)head_dim) : score_scale;
  const uint64_t offset = kv_seq - seq;
  for (uint64_t h = 0; h < heads; ++h) {
    const uint64_t kvh = h / group;
    for (uint64_t t = 0; t < seq; ++t) {
      const uint64_t position = offset + t;
      const uint64_t upper = causal ? position + 1 : kv_seq;
      const float *qv = q + t * q_dim + h * head_dim;
      float max = -INFINITY;
      for (uint64_t j = 0; j < upper; ++j) {
        const float *kv = k + j * kv_dim + kvh * head_dim;
        float dot = 0.0f;
        for (uint64_t d = 0; d < head_dim; ++d) dot += qv[d] * kv[d];
        scores[j] = dot * scale;
        max = fmaxf(max, scores[j]);
      }
      float sum = 0.0f;
      for (uint64_t j = 0; j < upper; ++j) {
        scores[j] = expf(scores[j] - max);
        sum += scores[j];
      }
      float *o = out + t * q_dim + h * head_dim;
      for (uint64_t d = 0; d < head_dim; ++d) {
        float acc = 0.0f;
        for (uint64_t j = 0; j < upper; ++j) acc += (scores[j] / sum) * v[j * kv_dim + kvh * head_dim + d];
        o[d] = acc;
      }
    }
  }
  return 0;
}

/* silu-mul (src/lib.rs:2592-2596): mul(silu(gate), up), silu(x) =
 * x * (1 / (1 + exp(-x))) (src/lib.rs:993-1004, 1077-1089). */
void or_silu_mul(const float *gate, const float *up, uint64_t n, float *out) {
  for (uint64_t i = 0; i < n; ++i) {
    const float g = gate[i];
    const float s = g * (1.0f / (1.0f + expf(-g)));
    out[i] = s * up[i];
  }
}

/* add / residual-add (src/lib.rs:1019-1075, 1128-1133): a + b, with b
 * either a's size or one row of `cols` broadcast over a's rows. */
int or_add(const float *a, uint64_t n, const float *b, uint64_t b_n, float *out) {
  if (b_n == 0 || n % b_n) return -1;
  for (uint64_t i = 0; i < n; ++i) out[i] = a[i] + b[i % b_n];
  return 0;
}
