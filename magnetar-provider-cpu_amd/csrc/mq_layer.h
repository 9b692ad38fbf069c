// Host launchers of the decoder-layer kernels (mq_layer.hip). They check
// nothing: the C-ABI layer validates shapes and sizes before calling.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mq {

// out[r][c] = x[r][c] * (1 / sqrt(mean_c(x[r]^2) + eps)) * w[r * w_stride + c]
// (w_stride 0 broadcasts one weight row).
void launch_rmsnorm(const float* x, uint64_t rows, uint64_t cols, const float* w, uint64_t w_stride, float eps,
                    float* out, hipStream_t stream);

// Rotates `dimension / 2` pairs in each of head_count blocks of every row by
// (position_offset + row) * scale * freq[pair]; out may equal x.
void launch_rope(const float* x, uint64_t rows, uint64_t cols, uint64_t head_count, uint64_t dimension, float scale,
                 uint64_t position_offset, int half_split, const float* freq, float* out, hipStream_t stream);

// Attention of seq query rows over the first key_count rows of k / v, with
// `part` = seq * heads * attention_chunks(key_count) * (2 + head_dim) f32 of
// scratch. head_dim must be 128 and heads / kv_heads one of 1, 2, 4, 8;
// returns false (nothing launched) otherwise.
uint64_t attention_chunks(uint64_t key_count);
bool launch_attention(const float* q, const float* k, const float* v, uint64_t seq, uint64_t key_count,
                      uint64_t heads, uint64_t head_dim, uint64_t kv_heads, int causal, float scale, float* part,
                      float* out, hipStream_t stream);

// dst[i] = src[i], i < n (the buffers must not overlap)
void launch_copy(const float* src, uint64_t n, float* dst, hipStream_t stream);

// dst[i] = value, i < n (a kernel, not a memset: safe to record in a graph)
void launch_fill(float* dst, uint64_t n, float value, hipStream_t stream);

void launch_silu_mul(const float* g, const float* u, uint64_t n, float* out, hipStream_t stream);
// out[i] = a[i] + b[i % b_n]
void launch_add(const float* a, uint64_t n, const float* b, uint64_t b_n, float* out, hipStream_t stream);

}  // namespace mq
