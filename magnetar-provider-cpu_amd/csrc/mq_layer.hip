// gfx950 kernels for the decoder-layer operators around the packed matmul:
// rmsnorm, rope, attention (split-key decode), silu-mul and add. All
// tensors are row-major f32 in device memory. Built with
// -ffp-contract=off: each multiply and add rounds separately, as in the
// reference's operators; reductions run in a fixed tree order, so results
// are deterministic, and differ from the reference's left-to-right sums
// only by rounding.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "mq_layer.h"

namespace mq {
namespace {

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// ---------------------------------------------------------------------------
// rmsnorm (src/lib.rs:348-402): one work-group of 256 threads per row. The
// sum of squares is a per-thread partial over a strided range, then a wave
// and a cross-wave tree; scale = 1 / sqrt(mean + eps) with correctly
// rounded sqrt and division; out = v * scale * w.
// ---------------------------------------------------------------------------
template <bool VEC4>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, uint64_t cols,
                                                      const float* __restrict__ w, uint64_t w_stride, float eps,
                                                      float* __restrict__ out) {
  __shared__ float part[4];
  const uint64_t row = blockIdx.x;
  const float* v = x + row * cols;
  const float* wv = w + row * w_stride;
  float* o = out + row * cols;
  float s = 0.0f;
  if (VEC4) {
#pragma unroll 4
    for (uint64_t c = 4 * threadIdx.x; c < cols; c += 1024) {
      const float4 a = *reinterpret_cast<const float4*>(v + c);
      s += a.x * a.x;
      s += a.y * a.y;
      s += a.z * a.z;
      s += a.w * a.w;
    }
  } else {
    for (uint64_t c = threadIdx.x; c < cols; c += 256) s += v[c] * v[c];
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  const float total = (part[0] + part[1]) + (part[2] + part[3]);
  const float scale = 1.0f / sqrtf(total / static_cast<float>(cols) + eps);
  if (VEC4) {
#pragma unroll 4
    for (uint64_t c = 4 * threadIdx.x; c < cols; c += 1024) {
      const float4 a = *reinterpret_cast<const float4*>(v + c);
      const float4 g = *reinterpret_cast<const float4*>(wv + c);
      *reinterpret_cast<float4*>(o + c) =
          make_float4(a.x * scale * g.x, a.y * scale * g.y, a.z * scale * g.z, a.w * scale * g.w);
    }
  } else {
    for (uint64_t c = threadIdx.x; c < cols; c += 256) o[c] = v[c] * scale * wv[c];
  }
}

// ---------------------------------------------------------------------------
// rope (src/lib.rs:616-687): one thread per (row, head, rotated pair),
// angle = position * freq[pair] (the frequency table comes from the host,
// computed with the platform's powf as the reference does). Columns past
// `dimension` in each head are not touched here: the launcher copies them
// when out is not x.
// ---------------------------------------------------------------------------
// (x and out may be the same buffer: each thread reads its pair, then writes it)
__global__ __launch_bounds__(256) void rope_kernel(const float* x, uint64_t rows, uint64_t cols,
                                                   uint64_t head_count, uint64_t dimension, float scale,
                                                   uint64_t position_offset, int half_split,
                                                   const float* __restrict__ freq, float* out) {
  const uint64_t head_width = cols / head_count, half = dimension / 2;
  const uint64_t t = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= rows * head_count * half) return;
  const uint64_t row = t / (head_count * half);
  const uint64_t rem = t - row * head_count * half;
  const uint64_t head = rem / half, p = rem - head * half;
  const uint64_t base = row * cols + head * head_width;
  const float position = static_cast<float>(position_offset + row) * scale;
  const float angle = position * freq[p];
  const float s = sinf(angle), c = cosf(angle);
  const uint64_t first = half_split ? base + p : base + 2 * p;
  const uint64_t second = half_split ? base + p + half : base + 2 * p + 1;
  const float a = x[first], b = x[second];
  out[first] = a * c - b * s;
  out[second] = a * s + b * c;
}

// ---------------------------------------------------------------------------
// Attention, split over keys (src/lib.rs:780-990). Work-group = 4 waves =
// one (kv head, chunk of 64 keys, query row); wave w takes the chunk's keys
// 16 w .. 16 w + 15, so a chunk's 64 KB of K and V rows are in flight at
// once over 4 waves.
//  Scores: lane (kk, s), kk = lane / 8, s = lane % 8, takes keys kk and
//   kk + 8 of the wave's 16 and dimensions 4 s + 32 i .. + 3 (i = 0..3), so
//   each group of 8 lanes reads one whole 512-byte key row in 128-byte
//   pieces; the 8 partial dots per key meet by three xor-shuffles.
//  Softmax partials per head over the chunk (wave g % 4 takes head g of the
//   group): m = max score, p = exp(s - m), l = sum p.
//  Values: lane owns dimensions 2 lane, 2 lane + 1 of the wave's 16 keys;
//   the 4 waves' sums meet in LDS in wave order.
// attention_combine_kernel merges the chunks of each (head, query row):
// out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c.
// Every sum is in a fixed order that depends only on the chunk, so the
// last row of a causal prefill equals the one-row decode step bit for bit.
// ---------------------------------------------------------------------------
constexpr int kChunk = 64;
constexpr int kWaveKeys = 16;

template <int GROUP, int HD>
__global__ __launch_bounds__(256) void attention_partial_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v, uint64_t seq,
    uint64_t key_count, uint64_t heads, uint64_t kv_heads, int causal, float scale,
    float* __restrict__ part) {
  static_assert(HD == 128, "one 512-byte row per key and head");
  __shared__ float s_lds[GROUP][kChunk];
  __shared__ float ml_lds[GROUP][2];
  __shared__ float o_lds[4][GROUP][HD];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, kk = lane >> 3, sl = lane & 7;
  const uint64_t kvh = blockIdx.x, chunk = blockIdx.y, t = blockIdx.z;
  const uint64_t chunks = gridDim.y;
  const uint64_t q_dim = heads * HD, kv_dim = kv_heads * HD;
  const uint64_t upper = causal ? key_count - seq + t + 1 : key_count;
  const uint64_t j0 = chunk * kChunk;
  const uint64_t jn = upper > j0 ? (upper - j0 < kChunk ? upper - j0 : kChunk) : 0;
  float* dst0 = part + ((t * heads + kvh * GROUP) * chunks + chunk) * (2 + HD);
  if (jn == 0) {  // uniform over the work-group: an empty chunk
    for (int e = threadIdx.x; e < GROUP * (2 + HD); e += 256) {
      const int g = e / (2 + HD), i = e % (2 + HD);
      dst0[g * chunks * (2 + HD) + i] = i == 0 ? -INFINITY : 0.0f;
    }
    return;
  }
  // scores of keys 16 w + kk and 16 w + 8 + kk
  float4 kv4[2][4];
  const float* kbase = k + kvh * HD + 4 * sl;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int jl = kWaveKeys * w + 8 * it + kk;
    const float* krow = kbase + (j0 + (static_cast<uint64_t>(jl) < jn ? jl : 0)) * kv_dim;
#pragma unroll
    for (int i = 0; i < 4; ++i) kv4[it][i] = *reinterpret_cast<const float4*>(krow + 32 * i);
  }
  const float* qrow = q + t * q_dim + kvh * GROUP * HD + 4 * sl;
#pragma unroll
  for (int g = 0; g < GROUP; ++g) {
    float4 qv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[i] = *reinterpret_cast<const float4*>(qrow + g * HD + 32 * i);
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      float d = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        d += qv[i].x * kv4[it][i].x;
        d += qv[i].y * kv4[it][i].y;
        d += qv[i].z * kv4[it][i].z;
        d += qv[i].w * kv4[it][i].w;
      }
      d += __shfl_xor(d, 1);
      d += __shfl_xor(d, 2);
      d += __shfl_xor(d, 4);
      const int jl = kWaveKeys * w + 8 * it + kk;
      if (sl == 0) s_lds[g][jl] = static_cast<uint64_t>(jl) < jn ? d * scale : -INFINITY;
    }
  }
  __syncthreads();
  const bool mine = static_cast<uint64_t>(lane) < jn;
  for (int g = w; g < GROUP; g += 4) {
    const float sc = s_lds[g][lane];
    const float m = wave_max(sc);
    const float p = mine ? expf(sc - m) : 0.0f;
    const float l = wave_sum(p);
    s_lds[g][lane] = p;  // each lane rewrites only its own entry
    if (lane == 0) {
      ml_lds[g][0] = m;
      ml_lds[g][1] = l;
    }
  }
  __syncthreads();
  // values of keys 16 w .. 16 w + 15 (rows past jn weigh 0 and read row j0)
  float2 vv[kWaveKeys];
  const float* vbase = v + kvh * HD + 2 * lane;
#pragma unroll
  for (int jj = 0; jj < kWaveKeys; ++jj) {
    const int jl = kWaveKeys * w + jj;
    vv[jj] = *reinterpret_cast<const float2*>(vbase + (j0 + (static_cast<uint64_t>(jl) < jn ? jl : 0)) * kv_dim);
  }
#pragma unroll
  for (int g = 0; g < GROUP; ++g) {
    float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (int jj = 0; jj < kWaveKeys; ++jj) {
      const float p = s_lds[g][kWaveKeys * w + jj];
      o0 += p * vv[jj].x;
      o1 += p * vv[jj].y;
    }
    *reinterpret_cast<float2*>(&o_lds[w][g][2 * lane]) = make_float2(o0, o1);
  }
  __syncthreads();
  // part layout: [t][head][chunk][2 + HD]
  for (int e = threadIdx.x; e < GROUP * HD; e += 256) {
    const int g = e / HD, d = e % HD;
    const float o = ((o_lds[0][g][d] + o_lds[1][g][d]) + o_lds[2][g][d]) + o_lds[3][g][d];
    dst0[g * chunks * (2 + HD) + 2 + d] = o;
  }
  if (threadIdx.x < GROUP) {
    dst0[threadIdx.x * chunks * (2 + HD)] = ml_lds[threadIdx.x][0];
    dst0[threadIdx.x * chunks * (2 + HD) + 1] = ml_lds[threadIdx.x][1];
  }
}

// One work-group of 4 waves per (head, query row). Every wave finds the
// maximum over the chunks; wave 0 writes the weights e^(m_c - M) to LDS and
// forms the denominator; wave w then adds chunks w, w + 4, ... for all HD
// dimensions (2 per lane), and the 4 sums meet in LDS in wave order. The
// first 16 chunks of each wave are loaded before the maximum is known.
template <int HD>
__global__ __launch_bounds__(256) void attention_combine_kernel(const float* __restrict__ part, uint64_t heads,
                                                              uint64_t chunks, float* __restrict__ out) {
  __shared__ float w_lds[1024];
  __shared__ float o_lds[4][HD];
  __shared__ float den_lds;
  const uint64_t h = blockIdx.x, t = blockIdx.y;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const float* base = part + (t * heads + h) * chunks * (2 + HD);
  // the wave's first 16 chunks' partial outputs are requested with the
  // chunk maxima (one memory round trip for up to 64 chunks = 4096 keys)
  constexpr int kPre = 16;
  const float* col = base + 2 + 2 * lane;
  float2 opre[kPre];
#pragma unroll
  for (int i = 0; i < kPre; ++i) {
    const uint64_t c = static_cast<uint64_t>(w) + 4 * i;
    opre[i] = *reinterpret_cast<const float2*>(col + (c < chunks ? c : 0) * (2 + HD));
  }
  float mx = -INFINITY;
  for (uint64_t c = lane; c < chunks; c += 64) mx = fmaxf(mx, base[c * (2 + HD)]);
  mx = wave_max(mx);
  if (w == 0) {
    float den = 0.0f;
    for (uint64_t c = lane; c < chunks; c += 64) {
      const float mc = base[c * (2 + HD)];
      const float e = mc == -INFINITY ? 0.0f : expf(mc - mx);
      w_lds[c] = e;
      den += e * base[c * (2 + HD) + 1];
    }
    den = wave_sum(den);
    if (lane == 0) den_lds = den;
  }
  __syncthreads();
  float n0 = 0.0f, n1 = 0.0f;
#pragma unroll
  for (int i = 0; i < kPre; ++i) {
    const uint64_t c = static_cast<uint64_t>(w) + 4 * i;
    if (c < chunks) {
      const float e = w_lds[c];
      n0 += e * opre[i].x;
      n1 += e * opre[i].y;
    }
  }
#pragma unroll 8
  for (uint64_t c = static_cast<uint64_t>(w) + 4 * kPre; c < chunks; c += 4) {
    const float2 o = *reinterpret_cast<const float2*>(col + c * (2 + HD));
    const float e = w_lds[c];
    n0 += e * o.x;
    n1 += e * o.y;
  }
  *reinterpret_cast<float2*>(&o_lds[w][2 * lane]) = make_float2(n0, n1);
  __syncthreads();
  if (threadIdx.x < HD) {
    const int d = threadIdx.x;
    const float num = ((o_lds[0][d] + o_lds[1][d]) + o_lds[2][d]) + o_lds[3][d];
    out[t * heads * HD + h * HD + d] = num / den_lds;
  }
}

// ---------------------------------------------------------------------------
// silu-mul (src/lib.rs:2592-2596, 993-1004): g * (1 / (1 + exp(-g))) * u.
// add (src/lib.rs:1019-1075): a + b[i % b_n].
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                       uint64_t n, float* __restrict__ out) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float x = g[i];
  const float s = x * (1.0f / (1.0f + expf(-x)));
  out[i] = s * u[i];
}

__global__ __launch_bounds__(256) void add_kernel(const float* __restrict__ a, uint64_t n,
                                                  const float* __restrict__ b, uint64_t b_n,
                                                  float* __restrict__ out) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = a[i] + b[i % b_n];
}

// kv-write: a plain copy of `n` floats (a kernel rather than a DMA copy:
// its launch costs a fraction of a blit's for the few-KB rows of a decode
// step)
__global__ __launch_bounds__(256) void copy_kernel(const float* __restrict__ src, uint64_t n,
                                                   float* __restrict__ dst) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

__global__ __launch_bounds__(256) void fill_kernel(float* __restrict__ dst, uint64_t n, float value) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = value;
}

unsigned blocks_for(uint64_t n, unsigned per) { return static_cast<unsigned>((n + per - 1) / per); }

}  // namespace

void launch_rmsnorm(const float* x, uint64_t rows, uint64_t cols, const float* w, uint64_t w_stride, float eps,
                    float* out, hipStream_t stream) {
  const bool vec4 = cols % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(w) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0;
  if (vec4)
    hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, x, cols, w,
                       w_stride, eps, out);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, x, cols, w,
                       w_stride, eps, out);
}

void launch_rope(const float* x, uint64_t rows, uint64_t cols, uint64_t head_count, uint64_t dimension, float scale,
                 uint64_t position_offset, int half_split, const float* freq, float* out, hipStream_t stream) {
  if (out != x && dimension < cols / head_count)
    (void)hipMemcpyAsync(out, x, rows * cols * sizeof(float), hipMemcpyDeviceToDevice, stream);
  const uint64_t n = rows * head_count * (dimension / 2);
  hipLaunchKernelGGL(rope_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream, x, rows, cols, head_count,
                     dimension, scale, position_offset, half_split, freq, out);
}

uint64_t attention_chunks(uint64_t key_count) { return (key_count + kChunk - 1) / kChunk; }

bool launch_attention(const float* q, const float* k, const float* v, uint64_t seq, uint64_t key_count,
                      uint64_t heads, uint64_t head_dim, uint64_t kv_heads, int causal, float scale, float* part,
                      float* out, hipStream_t stream) {
  if (head_dim != 128 || attention_chunks(key_count) > 1024) return false;
  const uint64_t group = heads / kv_heads, chunks = attention_chunks(key_count);
  dim3 grid(static_cast<unsigned>(kv_heads), static_cast<unsigned>(chunks), static_cast<unsigned>(seq));
  switch (group) {
#define X(G)                                                                                                   \
  case G:                                                                                                      \
    hipLaunchKernelGGL((attention_partial_kernel<G, 128>), grid, dim3(256), 0, stream, q, k, v, seq, key_count, \
                       heads, kv_heads, causal, scale, part);                                                  \
    break;
    X(1) X(2) X(4) X(8)
#undef X
    default:
      return false;
  }
  hipLaunchKernelGGL((attention_combine_kernel<128>), dim3(static_cast<unsigned>(heads), static_cast<unsigned>(seq)),
                     dim3(256), 0, stream, part, heads, chunks, out);
  return true;
}

void launch_silu_mul(const float* g, const float* u, uint64_t n, float* out, hipStream_t stream) {
  hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream, g, u, n, out);
}

void launch_add(const float* a, uint64_t n, const float* b, uint64_t b_n, float* out, hipStream_t stream) {
  hipLaunchKernelGGL(add_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream, a, n, b, b_n, out);
}

void launch_copy(const float* src, uint64_t n, float* dst, hipStream_t stream) {
  hipLaunchKernelGGL(copy_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream, src, n, dst);
}

void launch_fill(float* dst, uint64_t n, float value, hipStream_t stream) {
  hipLaunchKernelGGL(fill_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream, dst, n, value);
}

}  // namespace mq
