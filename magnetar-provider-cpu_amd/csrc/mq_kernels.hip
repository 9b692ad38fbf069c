// gfx950 kernels for the GGUF block-quantized matmul path: tile repack,
// bit-exact dequantization, int8 activation quantization, the decode GEMV
// and the MFMA prefill GEMM.
//
// Built with -ffp-contract=off: no multiply-add is fused unless written as
// fmaf, so the dequantizer reproduces the reference's separately rounded
// product and difference.
#include "mq_device.h"
#include "mq_launch.h"

namespace mq {

namespace {

__device__ inline uint4 ld16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ inline uint2 ld8(const uint8_t* p) { return *reinterpret_cast<const uint2*>(p); }

inline unsigned grid_for(uint64_t threads, unsigned block) {
  return static_cast<unsigned>((threads + block - 1) / block);
}

// ---------------------------------------------------------------------------
// Repack: checkpoint block order -> tiles of 8 rows (see mq_device.h).
// ---------------------------------------------------------------------------

__global__ void repack_q4k_kernel(const uint8_t* __restrict__ raw, uint64_t rows, uint64_t nb,
                                  uint8_t* __restrict__ tiled) {
  uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  if (t >= rows * nb * 9) return;
  uint64_t p = t % 9, rb = t / 9;
  uint64_t b = rb % nb, n = rb / nb;
  uint4 v = ld16(raw + rb * kQ4kBlockBytes + 16 * p);
  uint8_t* dst = tiled + (((n >> 3) * nb + b) * 9 + p) * 128 + (n & 7) * 16;
  *reinterpret_cast<uint4*>(dst) = v;
}

__global__ void repack_iq4xs_kernel(const uint8_t* __restrict__ raw, uint64_t rows, uint64_t nb,
                                    uint8_t* __restrict__ tiled) {
  uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  if (t >= rows * nb * 17) return;
  uint64_t q = t % 17, rb = t / 17;
  uint64_t b = rb % nb, n = rb / nb;
  uint2 v = ld8(raw + rb * kIq4xsBlockBytes + 8 * q);
  uint8_t* tile = tiled + ((n >> 3) * nb + b) * kIq4xsTileBytes;
  uint8_t* dst;
  if (q == 0) {
    dst = tile + (n & 7) * 8;
  } else {
    uint64_t o = 8 * (q - 1);
    dst = tile + 64 + (o >> 4) * 128 + (n & 7) * 16 + (o & 15);
  }
  *reinterpret_cast<uint2*>(dst) = v;
}

// ---------------------------------------------------------------------------
// Dequantization, one thread per (row, block, run): value = scale * q - min,
// product and difference each rounded once.
// ---------------------------------------------------------------------------

__device__ inline void store_run(float* out, uint64_t rows, uint64_t k, uint64_t n, uint64_t col0,
                                 int logical, const float (&v)[32]) {
  if (logical) {
    for (int i = 0; i < 32; ++i) out[(col0 + i) * rows + n] = v[i];
  } else {
    float4* o = reinterpret_cast<float4*>(out + n * k + col0);
    for (int i = 0; i < 8; ++i) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
  }
}

__global__ void dequantize_q4k_kernel(const uint8_t* __restrict__ tiled, uint64_t rows, uint64_t nb,
                                      int logical, float* __restrict__ out) {
  uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  if (t >= rows * nb * 8) return;
  int j = static_cast<int>(t % 8);
  uint64_t rb = t / 8, b = rb % nb, n = rb / nb;
  const uint8_t* tile = tiled + ((n >> 3) * nb + b) * kQ4kTileBytes + (n & 7) * 16;
  uint4 hdr = ld16(tile);
  int c = j >> 1, shift = 4 * (j & 1);
  uint4 q0 = ld16(tile + 128 * (1 + 2 * c));
  uint4 q1 = ld16(tile + 128 * (2 + 2 * c));
  Q4kSixBit six = q4k_six_bit(hdr);
  uint32_t sc, m;
  q4k_sc_m(six, j, sc, m);
  float d = half_bits(hdr.x), dmin = half_bits(hdr.x >> 16);
  float scale = d * static_cast<float>(sc);
  float mn = dmin * static_cast<float>(m);
  uint32_t words[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  float v[32];
  for (int i = 0; i < 32; ++i) {
    uint32_t qv = (byte_of(words[i >> 2], i & 3) >> shift) & 0xFu;
    float p = scale * static_cast<float>(qv);
    v[i] = p - mn;
  }
  store_run(out, rows, nb * 256, n, b * 256 + 32 * j, logical, v);
}

__global__ void dequantize_iq4xs_kernel(const uint8_t* __restrict__ tiled, uint64_t rows, uint64_t nb,
                                        int logical, float* __restrict__ out) {
  uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  if (t >= rows * nb * 8) return;
  int j = static_cast<int>(t % 8);
  uint64_t rb = t / 8, b = rb % nb, n = rb / nb;
  const uint8_t* tile = tiled + ((n >> 3) * nb + b) * kIq4xsTileBytes;
  uint2 hdr = ld8(tile + (n & 7) * 8);
  uint4 qq = ld16(tile + 64 + 128 * j + (n & 7) * 16);
  float scale = half_bits(hdr.x) * static_cast<float>(iq4xs_ls(hdr, j));
  uint32_t words[4] = {qq.x, qq.y, qq.z, qq.w};
  float v[32];
  for (int t4 = 0; t4 < 4; ++t4) {
    uint32_t lo = iq4_lookup4(words[t4] & 0x0F0F0F0Fu);
    uint32_t hi = iq4_lookup4((words[t4] >> 4) & 0x0F0F0F0Fu);
    for (int e = 0; e < 4; ++e) {
      float ql = static_cast<float>(static_cast<int8_t>(byte_of(lo, e)));
      float qh = static_cast<float>(static_cast<int8_t>(byte_of(hi, e)));
      v[4 * t4 + e] = scale * ql;
      v[16 + 4 * t4 + e] = scale * qh;
    }
  }
  store_run(out, rows, nb * 256, n, b * 256 + 32 * j, logical, v);
}

// ---------------------------------------------------------------------------
// Int8 activation quantization: 8 lanes per 32-value block, 4 values each.
// amax = max(0, max |x|) ignoring NaN; d = amax / 127 (correctly rounded);
// q = saturate(round_half_even(x / d)), NaN -> 0, 0 when amax == 0.
// ---------------------------------------------------------------------------

__device__ inline int sat_i8(float v) {
  if (v != v) return 0;
  v = fminf(fmaxf(v, -128.0f), 127.0f);
  return static_cast<int>(v);
}

__global__ void quantize_act_kernel(const float* __restrict__ x, uint64_t total,
                                    int8_t* __restrict__ values, float* __restrict__ scales,
                                    int32_t* __restrict__ sums, uint16_t* __restrict__ a16, int int8) {
  uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  bool active = t < total / 4;
  float4 v = active ? reinterpret_cast<const float4*>(x)[t] : make_float4(0.f, 0.f, 0.f, 0.f);
  float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  for (int o = 1; o < 8; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 8));
  amax = fmaxf(0.0f, amax);
  float d = amax / 127.0f;
  int q0 = 0, q1 = 0, q2 = 0, q3 = 0;
  if (amax != 0.0f) {
    q0 = sat_i8(rintf(v.x / d));
    q1 = sat_i8(rintf(v.y / d));
    q2 = sat_i8(rintf(v.z / d));
    q3 = sat_i8(rintf(v.w / d));
  }
  int hs = q0 + q1 + q2 + q3;
  hs += __shfl_xor(hs, 1, 8);
  hs += __shfl_xor(hs, 2, 8);
  if (!active) return;
  if (values) {
    uint32_t packed = (static_cast<uint32_t>(q0) & 0xFFu) | ((static_cast<uint32_t>(q1) & 0xFFu) << 8) |
                      ((static_cast<uint32_t>(q2) & 0xFFu) << 16) | (static_cast<uint32_t>(q3) << 24);
    reinterpret_cast<uint32_t*>(values)[t] = packed;
  }
  int sub = static_cast<int>(t & 7);
  uint64_t blk = t >> 3;
  if (scales && sub == 0) scales[blk] = d;
  if (sums && (sub & 3) == 0) sums[2 * blk + (sub >> 2)] = hs;
  if (a16) {
    float f0, f1, f2, f3;
    if (int8) {
      f0 = static_cast<float>(q0) * d;
      f1 = static_cast<float>(q1) * d;
      f2 = static_cast<float>(q2) * d;
      f3 = static_cast<float>(q3) * d;
    } else {
      f0 = v.x;
      f1 = v.y;
      f2 = v.z;
      f3 = v.w;
    }
    __half2 h01 = __floats2half2_rn(f0, f1), h23 = __floats2half2_rn(f2, f3);
    uint2 w;
    w.x = *reinterpret_cast<uint32_t*>(&h01);
    w.y = *reinterpret_cast<uint32_t*>(&h23);
    reinterpret_cast<uint2*>(a16)[t] = w;
  }
}

__global__ void activations_f16_kernel(const float* __restrict__ x, uint64_t total,
                                       uint16_t* __restrict__ a16) {
  uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  if (t >= total / 4) return;
  float4 v = reinterpret_cast<const float4*>(x)[t];
  __half2 h01 = __floats2half2_rn(v.x, v.y), h23 = __floats2half2_rn(v.z, v.w);
  uint2 w;
  w.x = *reinterpret_cast<uint32_t*>(&h01);
  w.y = *reinterpret_cast<uint32_t*>(&h23);
  reinterpret_cast<uint2*>(a16)[t] = w;
}

// ---------------------------------------------------------------------------
// Decode GEMV (m <= 8). One work-group per row group of 8 stored rows,
// `splits` waves per group. Lane = r + 8 * lam: row r of the group, blocks
// b = lam + 8 * (split + splits * i). Integer dots per run (v_dot4), scaled
// per run as d_act * scale_run, mins through the activation sums; lanes of
// a row reduced by shuffles, waves of a group through LDS in fixed order.
// ---------------------------------------------------------------------------

// y[m][row] = (acc - mins) [+ addend[m * addend_stride + row]]: the
// product rounded first, then the bias / residual added, as the reference's
// separate `add` does.
template <int M>
__device__ inline void reduce_and_store(float (&acc)[M], float (&mins)[M], uint64_t rows, float* y,
                                        const float* addend, uint64_t addend_stride) {
  __shared__ float red[8][M][8][2];
  const int lane = threadIdx.x & 63, s = threadIdx.x >> 6, S = blockDim.x >> 6;
  const int r = lane & 7, lam = lane >> 3;
#pragma unroll
  for (int m = 0; m < M; ++m) {
#pragma unroll
    for (int o = 8; o < 64; o <<= 1) {
      acc[m] += __shfl_xor(acc[m], o);
      mins[m] += __shfl_xor(mins[m], o);
    }
  }
  const uint64_t row = static_cast<uint64_t>(blockIdx.x) * 8 + r;
  if (S == 1) {
    if (lam == 0 && row < rows) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float v = acc[m] - mins[m];
        if (addend) v = v + addend[m * addend_stride + row];
        y[m * rows + row] = v;
      }
    }
    return;
  }
  if (lam == 0) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      red[s][m][r][0] = acc[m];
      red[s][m][r][1] = mins[m];
    }
  }
  __syncthreads();
  if (threadIdx.x < 8 && row < rows) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float a = 0.0f, mn = 0.0f;
      for (int i = 0; i < S; ++i) {
        a += red[i][m][threadIdx.x][0];
        mn += red[i][m][threadIdx.x][1];
      }
      float v = a - mn;
      if (addend) v = v + addend[m * addend_stride + row];
      y[m * rows + row] = v;
    }
  }
}

template <int M>
__global__ __launch_bounds__(512) void gemv_q4k_int8_kernel(
    const uint8_t* __restrict__ w, int nb, uint64_t rows, const int8_t* __restrict__ xv,
    const float* __restrict__ xs, const int32_t* __restrict__ xsum, float* __restrict__ y,
    const float* __restrict__ addend, uint64_t addend_stride) {
  const int lane = threadIdx.x & 63, s = threadIdx.x >> 6, S = blockDim.x >> 6;
  const int r = lane & 7, lam = lane >> 3;
  const uint64_t g = blockIdx.x;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  const int runs = nb * 8;
  float acc[M], mins[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = mins[m] = 0.0f;
  for (int b = lam + 8 * s; b < nb; b += 8 * S) {
    const uint8_t* tile = w + (g * nb + b) * kQ4kTileBytes + r * 16;
    uint4 hdr = ld16(tile);
    uint4 q[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) q[p] = ld16(tile + 128 * (p + 1));
    const float d = half_bits(hdr.x), dmin = half_bits(hdr.x >> 16);
    const Q4kSixBit six = q4k_six_bit(hdr);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint32_t sc0, m0, sc1, m1;
      q4k_sc_m(six, 2 * c, sc0, m0);
      q4k_sc_m(six, 2 * c + 1, sc1, m1);
      const float s0 = d * static_cast<float>(sc0), s1 = d * static_cast<float>(sc1);
      const float mn0 = dmin * static_cast<float>(m0), mn1 = dmin * static_cast<float>(m1);
      int dlo[M], dhi[M];
#pragma unroll
      for (int m = 0; m < M; ++m) dlo[m] = dhi[m] = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4 qq = q[2 * c + h];
        const uint32_t lo[4] = {qq.x & 0x0F0F0F0Fu, qq.y & 0x0F0F0F0Fu, qq.z & 0x0F0F0F0Fu,
                                qq.w & 0x0F0F0F0Fu};
        const uint32_t hi[4] = {(qq.x >> 4) & 0x0F0F0F0Fu, (qq.y >> 4) & 0x0F0F0F0Fu,
                                (qq.z >> 4) & 0x0F0F0F0Fu, (qq.w >> 4) & 0x0F0F0F0Fu};
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const uint8_t* xa = reinterpret_cast<const uint8_t*>(xv) + m * K + b * 256 + 64 * c + 16 * h;
          const uint4 x0 = ld16(xa), x1 = ld16(xa + 32);
          dlo[m] = sdot4(lo[0], x0.x, dlo[m]);
          dlo[m] = sdot4(lo[1], x0.y, dlo[m]);
          dlo[m] = sdot4(lo[2], x0.z, dlo[m]);
          dlo[m] = sdot4(lo[3], x0.w, dlo[m]);
          dhi[m] = sdot4(hi[0], x1.x, dhi[m]);
          dhi[m] = sdot4(hi[1], x1.y, dhi[m]);
          dhi[m] = sdot4(hi[2], x1.z, dhi[m]);
          dhi[m] = sdot4(hi[3], x1.w, dhi[m]);
        }
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const int u = b * 8 + 2 * c;
        const float2 da = *reinterpret_cast<const float2*>(xs + m * runs + u);
        const int4 sm = *reinterpret_cast<const int4*>(xsum + 2 * (m * runs + u));
        acc[m] = fmaf(static_cast<float>(dlo[m]), da.x * s0, acc[m]);
        acc[m] = fmaf(static_cast<float>(dhi[m]), da.y * s1, acc[m]);
        mins[m] = fmaf(da.x * mn0, static_cast<float>(sm.x + sm.y), mins[m]);
        mins[m] = fmaf(da.y * mn1, static_cast<float>(sm.z + sm.w), mins[m]);
      }
    }
  }
  reduce_and_store<M>(acc, mins, rows, y, addend, addend_stride);
}

template <int M>
__global__ __launch_bounds__(512) void gemv_iq4xs_int8_kernel(
    const uint8_t* __restrict__ w, int nb, uint64_t rows, const int8_t* __restrict__ xv,
    const float* __restrict__ xs, float* __restrict__ y, const float* __restrict__ addend,
    uint64_t addend_stride) {
  const int lane = threadIdx.x & 63, s = threadIdx.x >> 6, S = blockDim.x >> 6;
  const int r = lane & 7, lam = lane >> 3;
  const uint64_t g = blockIdx.x;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  const int runs = nb * 8;
  float acc[M], mins[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = mins[m] = 0.0f;
  for (int b = lam + 8 * s; b < nb; b += 8 * S) {
    const uint8_t* tile = w + (g * nb + b) * kIq4xsTileBytes;
    const uint2 hdr = ld8(tile + r * 8);
    uint4 q[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) q[p] = ld16(tile + 64 + 128 * p + r * 16);
    const float d = half_bits(hdr.x);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float sj = d * static_cast<float>(iq4xs_ls(hdr, j));
      const uint4 qq = q[j];
      const uint32_t lo[4] = {iq4_lookup4(qq.x & 0x0F0F0F0Fu), iq4_lookup4(qq.y & 0x0F0F0F0Fu),
                              iq4_lookup4(qq.z & 0x0F0F0F0Fu), iq4_lookup4(qq.w & 0x0F0F0F0Fu)};
      const uint32_t hi[4] = {iq4_lookup4((qq.x >> 4) & 0x0F0F0F0Fu), iq4_lookup4((qq.y >> 4) & 0x0F0F0F0Fu),
                              iq4_lookup4((qq.z >> 4) & 0x0F0F0F0Fu), iq4_lookup4((qq.w >> 4) & 0x0F0F0F0Fu)};
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint8_t* xa = reinterpret_cast<const uint8_t*>(xv) + m * K + b * 256 + 32 * j;
        const uint4 x0 = ld16(xa), x1 = ld16(xa + 16);
        int dot = sdot4(lo[0], x0.x, 0);
        dot = sdot4(lo[1], x0.y, dot);
        dot = sdot4(lo[2], x0.z, dot);
        dot = sdot4(lo[3], x0.w, dot);
        dot = sdot4(hi[0], x1.x, dot);
        dot = sdot4(hi[1], x1.y, dot);
        dot = sdot4(hi[2], x1.z, dot);
        dot = sdot4(hi[3], x1.w, dot);
        const float da = xs[m * runs + b * 8 + j];
        acc[m] = fmaf(static_cast<float>(dot), da * sj, acc[m]);
      }
    }
  }
  reduce_and_store<M>(acc, mins, rows, y, addend, addend_stride);
}

// ---------------------------------------------------------------------------
// Decode GEMV, row-per-lane form (m <= 4). A work-group owns 64 consecutive
// stored rows (8 row groups), one row per lane; its waves split the
// super-blocks (wave s takes b = s, s + S, ...). Every lane of a wave reads
// the same block of activations, so the int8 values, scales and sums come
// through scalar loads and the vector memory path carries weight bytes
// only. Partial sums meet in LDS and wave 0 adds them in wave order.
// ---------------------------------------------------------------------------

template <int M>
__device__ inline void reduce_waves_and_store(float (&acc)[M], float (&mins)[M], uint64_t rows, float* y,
                                              const float* addend, uint64_t addend_stride) {
  __shared__ float red[16][M][2][64];
  const int lane = threadIdx.x & 63, s = threadIdx.x >> 6, S = blockDim.x >> 6;
  const uint64_t row = static_cast<uint64_t>(blockIdx.x) * 64 + lane;
  if (S > 1) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      red[s][m][0][lane] = acc[m];
      red[s][m][1][lane] = mins[m];
    }
    __syncthreads();
    if (s != 0) return;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float a = red[0][m][0][lane], mn = red[0][m][1][lane];
      for (int i = 1; i < S; ++i) {
        a += red[i][m][0][lane];
        mn += red[i][m][1][lane];
      }
      acc[m] = a;
      mins[m] = mn;
    }
  }
  if (row >= rows) return;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float v = acc[m] - mins[m];
    if (addend) v = v + addend[m * addend_stride + row];
    y[m * rows + row] = v;
  }
}

template <int M>
__global__ __launch_bounds__(512) void gemv_rows_q4k_int8_kernel(
    const uint8_t* __restrict__ w, int nb, uint64_t rows, const int8_t* __restrict__ xv,
    const float* __restrict__ xs, const int32_t* __restrict__ xsum, float* __restrict__ y,
    const float* __restrict__ addend, uint64_t addend_stride) {
  const int lane = threadIdx.x & 63;
  const int s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = blockDim.x >> 6;
  const uint64_t g = static_cast<uint64_t>(blockIdx.x) * 8 + (lane >> 3);
  const bool live = g < (rows + 7) / 8;
  const int r = lane & 7;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  const int runs = nb * 8;
  float acc[M], mins[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = mins[m] = 0.0f;
  const uint8_t* base = w + g * nb * kQ4kTileBytes + r * 16;
  // Software pipeline: the next block's nine loads are issued before the
  // current block is computed.
  uint4 nhdr = make_uint4(0, 0, 0, 0), nq[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) nq[p] = make_uint4(0, 0, 0, 0);
  if (live && s < nb) {
    const uint8_t* tile = base + static_cast<uint64_t>(s) * kQ4kTileBytes;
    nhdr = ld16(tile);
#pragma unroll
    for (int p = 0; p < 8; ++p) nq[p] = ld16(tile + 128 * (p + 1));
  }
  for (int b = s; b < nb; b += S) {
    const uint4 hdr = nhdr;
    uint4 q[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) q[p] = nq[p];
    if (live && b + S < nb) {
      const uint8_t* tile = base + static_cast<uint64_t>(b + S) * kQ4kTileBytes;
      nhdr = ld16(tile);
#pragma unroll
      for (int p = 0; p < 8; ++p) nq[p] = ld16(tile + 128 * (p + 1));
    }
    const float d = half_bits(hdr.x), dmin = half_bits(hdr.x >> 16);
    const Q4kSixBit six = q4k_six_bit(hdr);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint32_t sc0, m0, sc1, m1;
      q4k_sc_m(six, 2 * c, sc0, m0);
      q4k_sc_m(six, 2 * c + 1, sc1, m1);
      const float s0 = d * static_cast<float>(sc0), s1 = d * static_cast<float>(sc1);
      const float mn0 = dmin * static_cast<float>(m0), mn1 = dmin * static_cast<float>(m1);
      int dlo[M], dhi[M];
#pragma unroll
      for (int m = 0; m < M; ++m) dlo[m] = dhi[m] = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4 qq = q[2 * c + h];
        const uint32_t lo[4] = {qq.x & 0x0F0F0F0Fu, qq.y & 0x0F0F0F0Fu, qq.z & 0x0F0F0F0Fu,
                                qq.w & 0x0F0F0F0Fu};
        const uint32_t hi[4] = {(qq.x >> 4) & 0x0F0F0F0Fu, (qq.y >> 4) & 0x0F0F0F0Fu,
                                (qq.z >> 4) & 0x0F0F0F0Fu, (qq.w >> 4) & 0x0F0F0F0Fu};
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const uint4* xa = reinterpret_cast<const uint4*>(xv + m * K + b * 256 + 64 * c + 16 * h);
          const uint4 x0 = xa[0], x1 = xa[2];
          dlo[m] = sdot4(lo[0], x0.x, dlo[m]);
          dlo[m] = sdot4(lo[1], x0.y, dlo[m]);
          dlo[m] = sdot4(lo[2], x0.z, dlo[m]);
          dlo[m] = sdot4(lo[3], x0.w, dlo[m]);
          dhi[m] = sdot4(hi[0], x1.x, dhi[m]);
          dhi[m] = sdot4(hi[1], x1.y, dhi[m]);
          dhi[m] = sdot4(hi[2], x1.z, dhi[m]);
          dhi[m] = sdot4(hi[3], x1.w, dhi[m]);
        }
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const int u = b * 8 + 2 * c;
        const float2 da = *reinterpret_cast<const float2*>(xs + m * runs + u);
        const int4 sm = *reinterpret_cast<const int4*>(xsum + 2 * (m * runs + u));
        acc[m] = fmaf(static_cast<float>(dlo[m]), da.x * s0, acc[m]);
        acc[m] = fmaf(static_cast<float>(dhi[m]), da.y * s1, acc[m]);
        mins[m] = fmaf(da.x * mn0, static_cast<float>(sm.x + sm.y), mins[m]);
        mins[m] = fmaf(da.y * mn1, static_cast<float>(sm.z + sm.w), mins[m]);
      }
    }
  }
  reduce_waves_and_store<M>(acc, mins, rows, y, addend, addend_stride);
}

template <int M>
__global__ __launch_bounds__(512) void gemv_rows_iq4xs_int8_kernel(
    const uint8_t* __restrict__ w, int nb, uint64_t rows, const int8_t* __restrict__ xv,
    const float* __restrict__ xs, float* __restrict__ y, const float* __restrict__ addend,
    uint64_t addend_stride) {
  const int lane = threadIdx.x & 63;
  const int s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = blockDim.x >> 6;
  const uint64_t g = static_cast<uint64_t>(blockIdx.x) * 8 + (lane >> 3);
  const bool live = g < (rows + 7) / 8;
  const int r = lane & 7;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  const int runs = nb * 8;
  float acc[M], mins[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = mins[m] = 0.0f;
  const uint8_t* base = w + g * nb * kIq4xsTileBytes;
  uint2 nhdr = make_uint2(0, 0);
  uint4 nq[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) nq[p] = make_uint4(0, 0, 0, 0);
  if (live && s < nb) {
    const uint8_t* tile = base + static_cast<uint64_t>(s) * kIq4xsTileBytes;
    nhdr = ld8(tile + r * 8);
#pragma unroll
    for (int p = 0; p < 8; ++p) nq[p] = ld16(tile + 64 + 128 * p + r * 16);
  }
  for (int b = s; b < nb; b += S) {
    const uint2 hdr = nhdr;
    uint4 q[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) q[p] = nq[p];
    if (live && b + S < nb) {
      const uint8_t* tile = base + static_cast<uint64_t>(b + S) * kIq4xsTileBytes;
      nhdr = ld8(tile + r * 8);
#pragma unroll
      for (int p = 0; p < 8; ++p) nq[p] = ld16(tile + 64 + 128 * p + r * 16);
    }
    const float d = half_bits(hdr.x);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float sj = d * static_cast<float>(iq4xs_ls(hdr, j));
      const uint4 qq = q[j];
      const uint32_t lo[4] = {iq4_lookup4(qq.x & 0x0F0F0F0Fu), iq4_lookup4(qq.y & 0x0F0F0F0Fu),
                              iq4_lookup4(qq.z & 0x0F0F0F0Fu), iq4_lookup4(qq.w & 0x0F0F0F0Fu)};
      const uint32_t hi[4] = {iq4_lookup4((qq.x >> 4) & 0x0F0F0F0Fu), iq4_lookup4((qq.y >> 4) & 0x0F0F0F0Fu),
                              iq4_lookup4((qq.z >> 4) & 0x0F0F0F0Fu), iq4_lookup4((qq.w >> 4) & 0x0F0F0F0Fu)};
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint4* xa = reinterpret_cast<const uint4*>(xv + m * K + b * 256 + 32 * j);
        const uint4 x0 = xa[0], x1 = xa[1];
        int dot = sdot4(lo[0], x0.x, 0);
        dot = sdot4(lo[1], x0.y, dot);
        dot = sdot4(lo[2], x0.z, dot);
        dot = sdot4(lo[3], x0.w, dot);
        dot = sdot4(hi[0], x1.x, dot);
        dot = sdot4(hi[1], x1.y, dot);
        dot = sdot4(hi[2], x1.z, dot);
        dot = sdot4(hi[3], x1.w, dot);
        const float da = xs[m * runs + b * 8 + j];
        acc[m] = fmaf(static_cast<float>(dot), da * sj, acc[m]);
      }
    }
  }
  reduce_waves_and_store<M>(acc, mins, rows, y, addend, addend_stride);
}

// ---------------------------------------------------------------------------
// Decode GEMV, row-per-lane with the activations staged in LDS (m <= 4).
// Same work split as above; the work-group first copies its activations
// (int8 values) into LDS together with two f32 per run, d_act and
// d_act * (s0 + s1), while the first block's weight loads are in flight.
// The block loop then reads them as LDS broadcasts. Per run the integer dot
// is scaled by the 6-bit scale in integer arithmetic (exact), so a block
// costs one f32 multiply-add per run for the scales and one for the mins,
// then one multiply by d and one by dmin.
// LDS bytes: m * (k + 8 * k / 32) for Q4_K, m * (k + 4 * k / 32) for IQ4_XS.
// ---------------------------------------------------------------------------

template <int TYPE, int M>
__device__ inline void stage_activations(const int8_t* __restrict__ xv, const float* __restrict__ xs,
                                         const int32_t* __restrict__ xsum, uint64_t K, uint8_t* lds) {
  const int runs = static_cast<int>(K / 32);
  const int n16 = static_cast<int>(M * K / 16);
  for (int i = threadIdx.x; i < n16; i += blockDim.x)
    reinterpret_cast<uint4*>(lds)[i] = reinterpret_cast<const uint4*>(xv)[i];
  float* rs = reinterpret_cast<float*>(lds + M * K);
  for (int i = threadIdx.x; i < M * runs; i += blockDim.x) {
    const float d = xs[i];
    if (TYPE == kTypeQ4K) {
      const int2 sm = reinterpret_cast<const int2*>(xsum)[i];
      rs[2 * i] = d;
      rs[2 * i + 1] = d * static_cast<float>(sm.x + sm.y);
    } else {
      rs[i] = d;
    }
  }
}

template <int M>
__global__ __launch_bounds__(1024) void gemv_lds_q4k_int8_kernel(
    const uint8_t* __restrict__ w, int nb, uint64_t rows, const int8_t* __restrict__ xv,
    const float* __restrict__ xs, const int32_t* __restrict__ xsum, float* __restrict__ y,
    const float* __restrict__ addend, uint64_t addend_stride) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = blockDim.x >> 6;
  const uint64_t g = static_cast<uint64_t>(blockIdx.x) * 8 + (lane >> 3);
  const bool live = g < (rows + 7) / 8;
  const int r = lane & 7;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  const int runs = nb * 8;
  const uint8_t* base = w + g * nb * kQ4kTileBytes + r * 16;
  uint4 nhdr = make_uint4(0, 0, 0, 0), nq[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) nq[p] = make_uint4(0, 0, 0, 0);
  if (live && s < nb) {
    const uint8_t* tile = base + static_cast<uint64_t>(s) * kQ4kTileBytes;
    nhdr = ld16(tile);
#pragma unroll
    for (int p = 0; p < 8; ++p) nq[p] = ld16(tile + 128 * (p + 1));
  }
  stage_activations<kTypeQ4K, M>(xv, xs, xsum, K, lds);
  __syncthreads();
  const float2* rs = reinterpret_cast<const float2*>(lds + M * K);
  float acc[M], mins[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = mins[m] = 0.0f;
  for (int b = s; b < nb; b += S) {
    const uint4 hdr = nhdr;
    uint4 q[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) q[p] = nq[p];
    if (live && b + S < nb) {
      const uint8_t* tile = base + static_cast<uint64_t>(b + S) * kQ4kTileBytes;
      nhdr = ld16(tile);
#pragma unroll
      for (int p = 0; p < 8; ++p) nq[p] = ld16(tile + 128 * (p + 1));
    }
    const Q4kSixBit six = q4k_six_bit(hdr);
    float accb[M], minb[M];
#pragma unroll
    for (int m = 0; m < M; ++m) accb[m] = minb[m] = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      int dlo[M], dhi[M];
#pragma unroll
      for (int m = 0; m < M; ++m) dlo[m] = dhi[m] = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4 qq = q[2 * c + h];
        const uint32_t lo[4] = {qq.x & 0x0F0F0F0Fu, qq.y & 0x0F0F0F0Fu, qq.z & 0x0F0F0F0Fu,
                                qq.w & 0x0F0F0F0Fu};
        const uint32_t hi[4] = {(qq.x >> 4) & 0x0F0F0F0Fu, (qq.y >> 4) & 0x0F0F0F0Fu,
                                (qq.z >> 4) & 0x0F0F0F0Fu, (qq.w >> 4) & 0x0F0F0F0Fu};
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const uint4* xa = reinterpret_cast<const uint4*>(lds + m * K + b * 256 + 64 * c + 16 * h);
          const uint4 x0 = xa[0], x1 = xa[2];
          dlo[m] = sdot4(lo[0], x0.x, dlo[m]);
          dlo[m] = sdot4(lo[1], x0.y, dlo[m]);
          dlo[m] = sdot4(lo[2], x0.z, dlo[m]);
          dlo[m] = sdot4(lo[3], x0.w, dlo[m]);
          dhi[m] = sdot4(hi[0], x1.x, dhi[m]);
          dhi[m] = sdot4(hi[1], x1.y, dhi[m]);
          dhi[m] = sdot4(hi[2], x1.z, dhi[m]);
          dhi[m] = sdot4(hi[3], x1.w, dhi[m]);
        }
      }
      uint32_t sc0, m0, sc1, m1;
      q4k_sc_m(six, 2 * c, sc0, m0);
      q4k_sc_m(six, 2 * c + 1, sc1, m1);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float2 r0 = rs[m * runs + b * 8 + 2 * c], r1 = rs[m * runs + b * 8 + 2 * c + 1];
        accb[m] = fmaf(static_cast<float>(__mul24(dlo[m], static_cast<int>(sc0))), r0.x, accb[m]);
        accb[m] = fmaf(static_cast<float>(__mul24(dhi[m], static_cast<int>(sc1))), r1.x, accb[m]);
        minb[m] = fmaf(static_cast<float>(m0), r0.y, minb[m]);
        minb[m] = fmaf(static_cast<float>(m1), r1.y, minb[m]);
      }
    }
    const float d = half_bits(hdr.x), dmin = half_bits(hdr.x >> 16);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      acc[m] = fmaf(d, accb[m], acc[m]);
      mins[m] = fmaf(dmin, minb[m], mins[m]);
    }
  }
  reduce_waves_and_store<M>(acc, mins, rows, y, addend, addend_stride);
}

template <int M>
__global__ __launch_bounds__(1024) void gemv_lds_iq4xs_int8_kernel(
    const uint8_t* __restrict__ w, int nb, uint64_t rows, const int8_t* __restrict__ xv,
    const float* __restrict__ xs, float* __restrict__ y, const float* __restrict__ addend,
    uint64_t addend_stride) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = blockDim.x >> 6;
  const uint64_t g = static_cast<uint64_t>(blockIdx.x) * 8 + (lane >> 3);
  const bool live = g < (rows + 7) / 8;
  const int r = lane & 7;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  const int runs = nb * 8;
  const uint8_t* base = w + g * nb * kIq4xsTileBytes;
  uint2 nhdr = make_uint2(0, 0);
  uint4 nq[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) nq[p] = make_uint4(0, 0, 0, 0);
  if (live && s < nb) {
    const uint8_t* tile = base + static_cast<uint64_t>(s) * kIq4xsTileBytes;
    nhdr = ld8(tile + r * 8);
#pragma unroll
    for (int p = 0; p < 8; ++p) nq[p] = ld16(tile + 64 + 128 * p + r * 16);
  }
  stage_activations<kTypeIq4Xs, M>(xv, xs, nullptr, K, lds);
  __syncthreads();
  const float* rs = reinterpret_cast<const float*>(lds + M * K);
  float acc[M], mins[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = mins[m] = 0.0f;
  for (int b = s; b < nb; b += S) {
    const uint2 hdr = nhdr;
    uint4 q[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) q[p] = nq[p];
    if (live && b + S < nb) {
      const uint8_t* tile = base + static_cast<uint64_t>(b + S) * kIq4xsTileBytes;
      nhdr = ld8(tile + r * 8);
#pragma unroll
      for (int p = 0; p < 8; ++p) nq[p] = ld16(tile + 64 + 128 * p + r * 16);
    }
    float accb[M];
#pragma unroll
    for (int m = 0; m < M; ++m) accb[m] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int ls = iq4xs_ls(hdr, j);
      const uint4 qq = q[j];
      const uint32_t lo[4] = {iq4_lookup4(qq.x & 0x0F0F0F0Fu), iq4_lookup4(qq.y & 0x0F0F0F0Fu),
                              iq4_lookup4(qq.z & 0x0F0F0F0Fu), iq4_lookup4(qq.w & 0x0F0F0F0Fu)};
      const uint32_t hi[4] = {iq4_lookup4((qq.x >> 4) & 0x0F0F0F0Fu), iq4_lookup4((qq.y >> 4) & 0x0F0F0F0Fu),
                              iq4_lookup4((qq.z >> 4) & 0x0F0F0F0Fu), iq4_lookup4((qq.w >> 4) & 0x0F0F0F0Fu)};
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint4* xa = reinterpret_cast<const uint4*>(lds + m * K + b * 256 + 32 * j);
        const uint4 x0 = xa[0], x1 = xa[1];
        int dot = sdot4(lo[0], x0.x, 0);
        dot = sdot4(lo[1], x0.y, dot);
        dot = sdot4(lo[2], x0.z, dot);
        dot = sdot4(lo[3], x0.w, dot);
        dot = sdot4(hi[0], x1.x, dot);
        dot = sdot4(hi[1], x1.y, dot);
        dot = sdot4(hi[2], x1.z, dot);
        dot = sdot4(hi[3], x1.w, dot);
        accb[m] = fmaf(static_cast<float>(__mul24(dot, ls)), rs[m * runs + b * 8 + j], accb[m]);
      }
    }
    const float d = half_bits(hdr.x);
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = fmaf(d, accb[m], acc[m]);
  }
  reduce_waves_and_store<M>(acc, mins, rows, y, addend, addend_stride);
}

// f32 activations: per run half, sum(q * x) and sum(x) in f32, then
// acc += scale * sum(q x) - min * sum(x).
__device__ inline float4 ldf4(const float* p) { return *reinterpret_cast<const float4*>(p); }

__device__ inline void dot_nibbles_f32(uint32_t bytes4, float4 x, float& dq, float& sx) {
  dq = fmaf(static_cast<float>(bytes4 & 0xFFu), x.x, dq);
  dq = fmaf(static_cast<float>((bytes4 >> 8) & 0xFFu), x.y, dq);
  dq = fmaf(static_cast<float>((bytes4 >> 16) & 0xFFu), x.z, dq);
  dq = fmaf(static_cast<float>(bytes4 >> 24), x.w, dq);
  sx += (x.x + x.y) + (x.z + x.w);
}

__device__ inline void dot_signed_f32(uint32_t bytes4, float4 x, float& dq) {
  dq = fmaf(static_cast<float>(static_cast<int8_t>(bytes4 & 0xFFu)), x.x, dq);
  dq = fmaf(static_cast<float>(static_cast<int8_t>((bytes4 >> 8) & 0xFFu)), x.y, dq);
  dq = fmaf(static_cast<float>(static_cast<int8_t>((bytes4 >> 16) & 0xFFu)), x.z, dq);
  dq = fmaf(static_cast<float>(static_cast<int8_t>(bytes4 >> 24)), x.w, dq);
}

template <int M>
__global__ __launch_bounds__(512) void gemv_q4k_f32_kernel(const uint8_t* __restrict__ w, int nb,
                                                           uint64_t rows, const float* __restrict__ x,
                                                           float* __restrict__ y, const float* __restrict__ addend,
                                                           uint64_t addend_stride) {
  const int lane = threadIdx.x & 63, s = threadIdx.x >> 6, S = blockDim.x >> 6;
  const int r = lane & 7, lam = lane >> 3;
  const uint64_t g = blockIdx.x;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  float acc[M], mins[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = mins[m] = 0.0f;
  for (int b = lam + 8 * s; b < nb; b += 8 * S) {
    const uint8_t* tile = w + (g * nb + b) * kQ4kTileBytes + r * 16;
    const uint4 hdr = ld16(tile);
    const float d = half_bits(hdr.x), dmin = half_bits(hdr.x >> 16);
    const Q4kSixBit six = q4k_six_bit(hdr);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint32_t sc0, m0, sc1, m1;
      q4k_sc_m(six, 2 * c, sc0, m0);
      q4k_sc_m(six, 2 * c + 1, sc1, m1);
      const float s0 = d * static_cast<float>(sc0), s1 = d * static_cast<float>(sc1);
      const float mn0 = dmin * static_cast<float>(m0), mn1 = dmin * static_cast<float>(m1);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4 qq = ld16(tile + 128 * (1 + 2 * c + h));
        const uint32_t wv[4] = {qq.x, qq.y, qq.z, qq.w};
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const float* xa = x + m * K + b * 256 + 64 * c + 16 * h;
          float dlo = 0.f, slo = 0.f, dhi = 0.f, shi = 0.f;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            dot_nibbles_f32(wv[t] & 0x0F0F0F0Fu, ldf4(xa + 4 * t), dlo, slo);
            dot_nibbles_f32((wv[t] >> 4) & 0x0F0F0F0Fu, ldf4(xa + 32 + 4 * t), dhi, shi);
          }
          acc[m] = fmaf(s0, dlo, acc[m]);
          acc[m] = fmaf(s1, dhi, acc[m]);
          mins[m] = fmaf(mn0, slo, mins[m]);
          mins[m] = fmaf(mn1, shi, mins[m]);
        }
      }
    }
  }
  reduce_and_store<M>(acc, mins, rows, y, addend, addend_stride);
}

template <int M>
__global__ __launch_bounds__(512) void gemv_iq4xs_f32_kernel(const uint8_t* __restrict__ w, int nb,
                                                             uint64_t rows, const float* __restrict__ x,
                                                             float* __restrict__ y, const float* __restrict__ addend,
                                                             uint64_t addend_stride) {
  const int lane = threadIdx.x & 63, s = threadIdx.x >> 6, S = blockDim.x >> 6;
  const int r = lane & 7, lam = lane >> 3;
  const uint64_t g = blockIdx.x;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  float acc[M], mins[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = mins[m] = 0.0f;
  for (int b = lam + 8 * s; b < nb; b += 8 * S) {
    const uint8_t* tile = w + (g * nb + b) * kIq4xsTileBytes;
    const uint2 hdr = ld8(tile + r * 8);
    const float d = half_bits(hdr.x);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float sj = d * static_cast<float>(iq4xs_ls(hdr, j));
      const uint4 qq = ld16(tile + 64 + 128 * j + r * 16);
      const uint32_t wv[4] = {qq.x, qq.y, qq.z, qq.w};
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float* xa = x + m * K + b * 256 + 32 * j;
        float dq = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          dot_signed_f32(iq4_lookup4(wv[t] & 0x0F0F0F0Fu), ldf4(xa + 4 * t), dq);
          dot_signed_f32(iq4_lookup4((wv[t] >> 4) & 0x0F0F0F0Fu), ldf4(xa + 16 + 4 * t), dq);
        }
        acc[m] = fmaf(sj, dq, acc[m]);
      }
    }
  }
  reduce_and_store<M>(acc, mins, rows, y, addend, addend_stride);
}

// ---------------------------------------------------------------------------
// Prefill GEMM on MFMA (v_mfma_f32_16x16x32_f16). Work-group tile 128 x 128,
// K-step 64 (one Q4_K quant chunk, two runs). 4 waves as 2 x 2, 64 x 64 each.
// Per K-step: the A tile (f16 activations) is copied to LDS; the B tile is
// dequantized once per work-group (f32 scale * q - min, rounded to f16) into
// LDS; each wave then runs 4 x 4 MFMAs per 32 of K.
// ---------------------------------------------------------------------------

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBN = 128, kBK = 64, kLdsK = kBK + 8;

__device__ inline uint32_t pack_f16x2(float a, float b) {
  __half2 h = __floats2half2_rn(a, b);
  return *reinterpret_cast<uint32_t*>(&h);
}

template <int TYPE>
__global__ __launch_bounds__(256) void gemm_kernel(const uint8_t* __restrict__ w, int nb, uint64_t rows,
                                                   uint64_t rows_padded, const uint16_t* __restrict__ a16,
                                                   uint64_t m_rows, float* __restrict__ y,
                                                   const float* __restrict__ addend, uint64_t addend_stride) {
  __shared__ __attribute__((aligned(16))) uint16_t As[kBM][kLdsK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[kBN][kLdsK];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const uint64_t m0 = static_cast<uint64_t>(blockIdx.y) * kBM;
  const uint64_t n0 = static_cast<uint64_t>(blockIdx.x) * kBN;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int ksteps = nb * 4;
  for (int kb = 0; kb < ksteps; ++kb) {
    // A tile: 128 rows x 64 halves, 16 B per chunk, 4 chunks per thread.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int idx = tid + 256 * i;
      int row = idx >> 3, ch = idx & 7;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (m0 + row < m_rows)
        v = *reinterpret_cast<const uint4*>(a16 + (m0 + row) * K + static_cast<uint64_t>(kb) * kBK + ch * 8);
      *reinterpret_cast<uint4*>(&As[row][ch * 8]) = v;
    }
    // B tile: thread -> (row nl, half h) dequantizes 32 weights.
    {
      const int nl = tid >> 1, h = tid & 1;
      const uint64_t n = n0 + nl;
      const int b = kb >> 2, c = kb & 3;
      uint32_t out[16];
      if (n < rows_padded) {
        if (TYPE == kTypeQ4K) {
          const uint8_t* tile = w + ((n >> 3) * nb + b) * kQ4kTileBytes + (n & 7) * 16;
          const uint4 hdr = ld16(tile);
          const uint4 qq = ld16(tile + 128 * (1 + 2 * c + h));
          const Q4kSixBit six = q4k_six_bit(hdr);
          uint32_t sc0, mm0, sc1, mm1;
          q4k_sc_m(six, 2 * c, sc0, mm0);
          q4k_sc_m(six, 2 * c + 1, sc1, mm1);
          const float d = half_bits(hdr.x), dmin = half_bits(hdr.x >> 16);
          const float s0 = d * static_cast<float>(sc0), s1 = d * static_cast<float>(sc1);
          const float mn0 = dmin * static_cast<float>(mm0), mn1 = dmin * static_cast<float>(mm1);
          const uint32_t wv[4] = {qq.x, qq.y, qq.z, qq.w};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint32_t lo = wv[t] & 0x0F0F0F0Fu, hi = (wv[t] >> 4) & 0x0F0F0F0Fu;
            out[2 * t] = pack_f16x2(fmaf(s0, static_cast<float>(lo & 0xFFu), -mn0),
                                    fmaf(s0, static_cast<float>((lo >> 8) & 0xFFu), -mn0));
            out[2 * t + 1] = pack_f16x2(fmaf(s0, static_cast<float>((lo >> 16) & 0xFFu), -mn0),
                                        fmaf(s0, static_cast<float>(lo >> 24), -mn0));
            out[8 + 2 * t] = pack_f16x2(fmaf(s1, static_cast<float>(hi & 0xFFu), -mn1),
                                        fmaf(s1, static_cast<float>((hi >> 8) & 0xFFu), -mn1));
            out[8 + 2 * t + 1] = pack_f16x2(fmaf(s1, static_cast<float>((hi >> 16) & 0xFFu), -mn1),
                                            fmaf(s1, static_cast<float>(hi >> 24), -mn1));
          }
        } else {
          const int j = 2 * c + h;
          const uint8_t* tile = w + ((n >> 3) * nb + b) * kIq4xsTileBytes;
          const uint2 hdr = ld8(tile + (n & 7) * 8);
          const uint4 qq = ld16(tile + 64 + 128 * j + (n & 7) * 16);
          const float sj = half_bits(hdr.x) * static_cast<float>(iq4xs_ls(hdr, j));
          const uint32_t wv[4] = {qq.x, qq.y, qq.z, qq.w};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint32_t lo = iq4_lookup4(wv[t] & 0x0F0F0F0Fu);
            const uint32_t hi = iq4_lookup4((wv[t] >> 4) & 0x0F0F0F0Fu);
            out[2 * t] = pack_f16x2(sj * static_cast<float>(static_cast<int8_t>(lo & 0xFFu)),
                                    sj * static_cast<float>(static_cast<int8_t>((lo >> 8) & 0xFFu)));
            out[2 * t + 1] = pack_f16x2(sj * static_cast<float>(static_cast<int8_t>((lo >> 16) & 0xFFu)),
                                        sj * static_cast<float>(static_cast<int8_t>(lo >> 24)));
            out[8 + 2 * t] = pack_f16x2(sj * static_cast<float>(static_cast<int8_t>(hi & 0xFFu)),
                                        sj * static_cast<float>(static_cast<int8_t>((hi >> 8) & 0xFFu)));
            out[8 + 2 * t + 1] = pack_f16x2(sj * static_cast<float>(static_cast<int8_t>((hi >> 16) & 0xFFu)),
                                            sj * static_cast<float>(static_cast<int8_t>(hi >> 24)));
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) out[i] = 0;
      }
      // Q4_K: run 2c weights 16h..16h+15 at k = 16h, run 2c+1 at k = 32 + 16h.
      // IQ4_XS: run 2c+h weights 0..15 at k = 32h, 16..31 at k = 32h + 16.
      const int k_lo = TYPE == kTypeQ4K ? 16 * h : 32 * h;
      const int k_hi = TYPE == kTypeQ4K ? 32 + 16 * h : 32 * h + 16;
      uint4* dlo = reinterpret_cast<uint4*>(&Bs[nl][k_lo]);
      uint4* dhi = reinterpret_cast<uint4*>(&Bs[nl][k_hi]);
      dlo[0] = make_uint4(out[0], out[1], out[2], out[3]);
      dlo[1] = make_uint4(out[4], out[5], out[6], out[7]);
      dhi[0] = make_uint4(out[8], out[9], out[10], out[11]);
      dhi[1] = make_uint4(out[12], out[13], out[14], out[15]);
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      half8 af[4], bf[4];
      const int koff = kk + 8 * (lane >> 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = *reinterpret_cast<const half8*>(&As[wm + 16 * i + (lane & 15)][koff]);
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = *reinterpret_cast<const half8*>(&Bs[wn + 16 * j + (lane & 15)][koff]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
  // D layout: lane holds column (lane & 15), rows 4 * (lane >> 4) + e.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint64_t col = n0 + wn + 16 * j + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint64_t row = m0 + wm + 16 * i + 4 * (lane >> 4) + e;
        if (row < m_rows && col < rows) {
          float v = acc[i][j][e];
          if (addend) v = v + addend[row * addend_stride + col];
          y[row * rows + col] = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Prefill GEMM, register-B form (v_mfma_f32_16x16x32_f16). A work-group of
// 4 waves covers MF*16 activation rows x 4*NF*16 weight rows; each wave owns
// NF*16 weight rows for the whole K loop and dequantizes its own B
// fragments from the tiled bytes straight into MFMA operand registers (f32
// scale * q - min, rounded once to f16), so B never touches LDS. The f16
// activation tile is the only LDS traffic: double-buffered, one barrier per
// 64-wide K-step (one Q4_K quant chunk = two runs).
//
// Operand lanes: lane = i + 16 * kq holds rows/columns i and k = 8 kq .. 8 kq + 7
// of the 32-wide MFMA K, for A and B alike; the weight bytes 8 kq .. 8 kq + 7
// of a chunk give run 2c's k-slot (low nibbles) and run 2c+1's (high).
// ---------------------------------------------------------------------------

template <int TYPE, int MF, int NF>
__global__ __launch_bounds__(256) void gemm_rb_kernel(const uint8_t* __restrict__ w, int nb, uint64_t rows,
                                                      uint64_t rows_padded, const uint16_t* __restrict__ a16,
                                                      uint64_t m_rows, float* __restrict__ y,
                                                      const float* __restrict__ addend, uint64_t addend_stride) {
  constexpr int BM = MF * 16;
  constexpr int LDK = kBK + 8;  // halves per LDS row (16-byte pad)
  constexpr int A_CHUNKS = BM * kBK / 8 / 256;  // 16-byte chunks per thread per K-step
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM][LDK];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int li = lane & 15, kq = lane >> 4;
  const uint64_t m0 = static_cast<uint64_t>(blockIdx.y) * BM;
  const uint64_t n0 = static_cast<uint64_t>(blockIdx.x) * (4 * NF * 16) + static_cast<uint64_t>(wave) * NF * 16;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  const int ksteps = nb * 4;

  floatx4 acc[MF][NF];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int f = 0; f < NF; ++f) acc[i][f] = floatx4{0.f, 0.f, 0.f, 0.f};

  // this lane's weight row per fragment
  const uint8_t* wrow[NF];
  bool wlive[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const uint64_t n = n0 + 16 * f + li;
    wlive[f] = n < rows_padded;
    const uint64_t nn = wlive[f] ? n : 0;
    wrow[f] = w + (nn >> 3) * nb * tile_bytes(TYPE) + (nn & 7) * (TYPE == kTypeQ4K ? 16 : 8);
  }

  auto load_a = [&](int kb, uint4 (&regs)[A_CHUNKS]) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int idx = tid + 256 * i, row = idx >> 3, ch = idx & 7;
      regs[i] = make_uint4(0, 0, 0, 0);
      if (m0 + row < m_rows)
        regs[i] = *reinterpret_cast<const uint4*>(a16 + (m0 + row) * K + static_cast<uint64_t>(kb) * kBK + ch * 8);
    }
  };
  auto store_a = [&](int buf, const uint4 (&regs)[A_CHUNKS]) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int idx = tid + 256 * i, row = idx >> 3, ch = idx & 7;
      *reinterpret_cast<uint4*>(&As[buf][row][ch * 8]) = regs[i];
    }
  };

  // raw B bytes for one K-step: Q4_K: 8 quant bytes per fragment (+ the
  // 16-byte header, reloaded at each new super-block); IQ4_XS: 8 index bytes
  // of each of the two runs (+ the 8-byte header).
  uint4 hdr[NF];
  uint2 qa[NF], qb[NF];
  auto load_b = [&](int kb) {
    const int b = kb >> 2, c = kb & 3;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint8_t* tile = wrow[f] + static_cast<uint64_t>(b) * tile_bytes(TYPE);
      if (!wlive[f]) {
        qa[f] = qb[f] = make_uint2(0, 0);
        if (c == 0) hdr[f] = make_uint4(0, 0, 0, 0);
        continue;
      }
      if (TYPE == kTypeQ4K) {
        if (c == 0) hdr[f] = ld16(tile);
        qa[f] = ld8(tile + 128 * (1 + 2 * c + (kq >> 1)) + 8 * (kq & 1));
      } else {
        if (c == 0) {
          const uint2 h = ld8(tile);
          hdr[f] = make_uint4(h.x, h.y, 0, 0);
        }
        // wrow points at this row's 8 header bytes; the quant planes start
        // 64 bytes into the tile, 16 bytes per row.
        const int rsub = static_cast<int>((n0 + 16 * f + li) & 7);
        const uint8_t* planes = tile - rsub * 8 + 64 + rsub * 16 + 8 * (kq & 1);
        qa[f] = ld8(planes + 128 * (2 * c));
        qb[f] = ld8(planes + 128 * (2 * c + 1));
      }
    }
  };

  uint4 areg[A_CHUNKS];
  load_a(0, areg);
  store_a(0, areg);
  load_b(0);
  __syncthreads();

  for (int kb = 0; kb < ksteps; ++kb) {
    const int buf = kb & 1;
    const int c = kb & 3;
    // dequantize this step's B fragments into operand registers
    half8 bop[2][NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      if (TYPE == kTypeQ4K) {
        const Q4kSixBit six = q4k_six_bit(hdr[f]);
        uint32_t sc0, mm0, sc1, mm1;
        q4k_sc_m(six, 2 * c, sc0, mm0);
        q4k_sc_m(six, 2 * c + 1, sc1, mm1);
        const float d = half_bits(hdr[f].x), dmin = half_bits(hdr[f].x >> 16);
        const float s0 = d * static_cast<float>(sc0), s1 = d * static_cast<float>(sc1);
        const float n0m = -(dmin * static_cast<float>(mm0)), n1m = -(dmin * static_cast<float>(mm1));
        uint32_t lo[2] = {qa[f].x & 0x0F0F0F0Fu, qa[f].y & 0x0F0F0F0Fu};
        uint32_t hi[2] = {(qa[f].x >> 4) & 0x0F0F0F0Fu, (qa[f].y >> 4) & 0x0F0F0F0Fu};
        uint32_t p0[4], p1[4];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          p0[2 * t] = pack_f16x2(fmaf(s0, static_cast<float>(lo[t] & 0xFFu), n0m),
                                 fmaf(s0, static_cast<float>((lo[t] >> 8) & 0xFFu), n0m));
          p0[2 * t + 1] = pack_f16x2(fmaf(s0, static_cast<float>((lo[t] >> 16) & 0xFFu), n0m),
                                     fmaf(s0, static_cast<float>(lo[t] >> 24), n0m));
          p1[2 * t] = pack_f16x2(fmaf(s1, static_cast<float>(hi[t] & 0xFFu), n1m),
                                 fmaf(s1, static_cast<float>((hi[t] >> 8) & 0xFFu), n1m));
          p1[2 * t + 1] = pack_f16x2(fmaf(s1, static_cast<float>((hi[t] >> 16) & 0xFFu), n1m),
                                     fmaf(s1, static_cast<float>(hi[t] >> 24), n1m));
        }
        bop[0][f] = *reinterpret_cast<half8*>(p0);
        bop[1][f] = *reinterpret_cast<half8*>(p1);
      } else {
        const uint2 h2 = make_uint2(hdr[f].x, hdr[f].y);
        const float d = half_bits(h2.x);
        const float sa = d * static_cast<float>(iq4xs_ls(h2, 2 * c));
        const float sb = d * static_cast<float>(iq4xs_ls(h2, 2 * c + 1));
        const int sh = 4 * (kq >> 1);  // low nibbles hold weights 0..15, high 16..31
        uint32_t ia[2] = {iq4_lookup4((qa[f].x >> sh) & 0x0F0F0F0Fu), iq4_lookup4((qa[f].y >> sh) & 0x0F0F0F0Fu)};
        uint32_t ib[2] = {iq4_lookup4((qb[f].x >> sh) & 0x0F0F0F0Fu), iq4_lookup4((qb[f].y >> sh) & 0x0F0F0F0Fu)};
        uint32_t p0[4], p1[4];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          p0[2 * t] = pack_f16x2(sa * static_cast<float>(static_cast<int8_t>(ia[t] & 0xFFu)),
                                 sa * static_cast<float>(static_cast<int8_t>((ia[t] >> 8) & 0xFFu)));
          p0[2 * t + 1] = pack_f16x2(sa * static_cast<float>(static_cast<int8_t>((ia[t] >> 16) & 0xFFu)),
                                     sa * static_cast<float>(static_cast<int8_t>(ia[t] >> 24)));
          p1[2 * t] = pack_f16x2(sb * static_cast<float>(static_cast<int8_t>(ib[t] & 0xFFu)),
                                 sb * static_cast<float>(static_cast<int8_t>((ib[t] >> 8) & 0xFFu)));
          p1[2 * t + 1] = pack_f16x2(sb * static_cast<float>(static_cast<int8_t>((ib[t] >> 16) & 0xFFu)),
                                     sb * static_cast<float>(static_cast<int8_t>(ib[t] >> 24)));
        }
        bop[0][f] = *reinterpret_cast<half8*>(p0);
        bop[1][f] = *reinterpret_cast<half8*>(p1);
      }
    }
    // prefetch the next step's A tile and B bytes
    const bool more = kb + 1 < ksteps;
    if (more) {
      load_a(kb + 1, areg);
      load_b(kb + 1);
    }
    // 2 runs x MF x NF MFMAs from the current A buffer
#pragma unroll
    for (int r = 0; r < 2; ++r) {
#pragma unroll
      for (int i = 0; i < MF; ++i) {
        const half8 af = *reinterpret_cast<const half8*>(&As[buf][16 * i + li][32 * r + 8 * kq]);
#pragma unroll
        for (int f = 0; f < NF; ++f)
          acc[i][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bop[r][f], acc[i][f], 0, 0, 0);
      }
    }
    if (more) store_a(buf ^ 1, areg);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < MF; ++i) {
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint64_t col = n0 + 16 * f + li;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint64_t row = m0 + 16 * i + 4 * kq + e;
        if (row < m_rows && col < rows) {
          float v = acc[i][f][e];
          if (addend) v = v + addend[row * addend_stride + col];
          y[row * rows + col] = v;
        }
      }
    }
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------

void launch_repack(int type, const uint8_t* raw, uint64_t rows, uint64_t nb, uint8_t* tiled,
                   hipStream_t stream) {
  if (type == kTypeQ4K) {
    uint64_t threads = rows * nb * 9;
    hipLaunchKernelGGL(repack_q4k_kernel, dim3(grid_for(threads, 256)), dim3(256), 0, stream, raw, rows, nb,
                       tiled);
  } else {
    uint64_t threads = rows * nb * 17;
    hipLaunchKernelGGL(repack_iq4xs_kernel, dim3(grid_for(threads, 256)), dim3(256), 0, stream, raw, rows,
                       nb, tiled);
  }
}

void launch_dequantize(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, int logical, float* out,
                       hipStream_t stream) {
  uint64_t threads = rows * nb * 8;
  if (type == kTypeQ4K)
    hipLaunchKernelGGL(dequantize_q4k_kernel, dim3(grid_for(threads, 256)), dim3(256), 0, stream, tiled, rows,
                       nb, logical, out);
  else
    hipLaunchKernelGGL(dequantize_iq4xs_kernel, dim3(grid_for(threads, 256)), dim3(256), 0, stream, tiled,
                       rows, nb, logical, out);
}

void launch_quantize_activations(const float* x, uint64_t m, uint64_t k, int8_t* values, float* scales,
                                 int32_t* sums, uint16_t* a16, int int8, hipStream_t stream) {
  uint64_t total = m * k;
  hipLaunchKernelGGL(quantize_act_kernel, dim3(grid_for(total / 4, 256)), dim3(256), 0, stream, x, total,
                     values, scales, sums, a16, int8);
}

void launch_activations_f16(const float* x, uint64_t m, uint64_t k, uint16_t* a16, hipStream_t stream) {
  uint64_t total = m * k;
  hipLaunchKernelGGL(activations_f16_kernel, dim3(grid_for(total / 4, 256)), dim3(256), 0, stream, x, total,
                     a16);
}

int gemv_default_splits(uint64_t rows, uint64_t nb, uint64_t m, int variant) {
  if (variant == 0) variant = m <= 4 ? 3 : 1;
  if (variant >= 2) {
    // waves per 64-row group: split the super-blocks, at least one each
    int splits = 1;
    while (splits < 8 && static_cast<uint64_t>(2 * splits) <= nb) splits *= 2;
    return splits;
  }
  const uint64_t groups = (rows + 7) / 8;
  int splits = 1;
  while (splits < 8 && groups * splits < 4096 && 8 * (2 * splits) <= nb) splits *= 2;
  return splits;
}

#define MQ_GEMV_CASES(X) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8)

void launch_gemv_int8(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, const int8_t* values,
                      const float* scales, const int32_t* sums, uint64_t m, float* y, const float* addend,
                      uint64_t addend_stride, int splits, int variant, hipStream_t stream) {
  const int inb = static_cast<int>(nb);
  const size_t lds_need = type == kTypeQ4K ? m * nb * 256 + m * nb * 8 * 8 : m * nb * 256 + m * nb * 8 * 4;
  if (variant == 0) variant = m <= 4 ? (lds_need <= 65536 ? 3 : 2) : 1;
  if (variant == 3 && m <= 4 && lds_need <= 65536) {
    dim3 grid(static_cast<unsigned>((rows + 63) / 64)), block(64 * splits);
    if (type == kTypeQ4K) {
      switch (m) {
#define X(MM)                                                                                         \
  case MM:                                                                                            \
    hipLaunchKernelGGL(gemv_lds_q4k_int8_kernel<MM>, grid, block, lds_need, stream, tiled, inb, rows, \
                       values, scales, sums, y, addend, addend_stride);                               \
    break;
        X(1) X(2) X(3) X(4)
#undef X
        default:
          break;
      }
    } else {
      switch (m) {
#define X(MM)                                                                                           \
  case MM:                                                                                              \
    hipLaunchKernelGGL(gemv_lds_iq4xs_int8_kernel<MM>, grid, block, lds_need, stream, tiled, inb, rows, \
                       values, scales, y, addend, addend_stride);                                       \
    break;
        X(1) X(2) X(3) X(4)
#undef X
        default:
          break;
      }
    }
    return;
  }
  if (variant >= 2 && m <= 4) {
    dim3 grid(static_cast<unsigned>((rows + 63) / 64)), block(64 * splits);
    if (type == kTypeQ4K) {
      switch (m) {
#define X(MM)                                                                                            \
  case MM:                                                                                               \
    hipLaunchKernelGGL(gemv_rows_q4k_int8_kernel<MM>, grid, block, 0, stream, tiled, inb, rows, values, \
                       scales, sums, y, addend, addend_stride);                                          \
    break;
        X(1) X(2) X(3) X(4)
#undef X
        default:
          break;
      }
    } else {
      switch (m) {
#define X(MM)                                                                                              \
  case MM:                                                                                                 \
    hipLaunchKernelGGL(gemv_rows_iq4xs_int8_kernel<MM>, grid, block, 0, stream, tiled, inb, rows, values, \
                       scales, y, addend, addend_stride);                                                  \
    break;
        X(1) X(2) X(3) X(4)
#undef X
        default:
          break;
      }
    }
    return;
  }
  dim3 grid(static_cast<unsigned>((rows + 7) / 8)), block(64 * splits);
  if (type == kTypeQ4K) {
    switch (m) {
#define X(MM)                                                                                           \
  case MM:                                                                                              \
    hipLaunchKernelGGL(gemv_q4k_int8_kernel<MM>, grid, block, 0, stream, tiled, inb, rows, values, scales, \
                       sums, y, addend, addend_stride);                                                 \
    break;
      MQ_GEMV_CASES(X)
#undef X
      default:
        break;
    }
  } else {
    switch (m) {
#define X(MM)                                                                                             \
  case MM:                                                                                                \
    hipLaunchKernelGGL(gemv_iq4xs_int8_kernel<MM>, grid, block, 0, stream, tiled, inb, rows, values, scales, \
                       y, addend, addend_stride);                                                         \
    break;
      MQ_GEMV_CASES(X)
#undef X
      default:
        break;
    }
  }
}

void launch_gemv_f32(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, const float* x, uint64_t m,
                     float* y, const float* addend, uint64_t addend_stride, int splits, hipStream_t stream) {
  dim3 grid(static_cast<unsigned>((rows + 7) / 8)), block(64 * splits);
  const int inb = static_cast<int>(nb);
  if (type == kTypeQ4K) {
    switch (m) {
#define X(MM)                                                                                       \
  case MM:                                                                                          \
    hipLaunchKernelGGL(gemv_q4k_f32_kernel<MM>, grid, block, 0, stream, tiled, inb, rows, x, y, addend, \
                       addend_stride);                                                            \
    break;
      MQ_GEMV_CASES(X)
#undef X
      default:
        break;
    }
  } else {
    switch (m) {
#define X(MM)                                                                                         \
  case MM:                                                                                            \
    hipLaunchKernelGGL(gemv_iq4xs_f32_kernel<MM>, grid, block, 0, stream, tiled, inb, rows, x, y, addend, \
                       addend_stride);                                                              \
    break;
      MQ_GEMV_CASES(X)
#undef X
      default:
        break;
    }
  }
}

namespace {

template <int MF, int NF>
void launch_gemm_rb(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, const uint16_t* a16, uint64_t m,
                    float* y, const float* addend, uint64_t addend_stride, hipStream_t stream) {
  const uint64_t rows_padded = (rows + 7) / 8 * 8;
  const uint64_t bn = 4 * NF * 16, bm = MF * 16;
  dim3 grid(static_cast<unsigned>((rows + bn - 1) / bn), static_cast<unsigned>((m + bm - 1) / bm));
  if (type == kTypeQ4K)
    hipLaunchKernelGGL((gemm_rb_kernel<kTypeQ4K, MF, NF>), grid, dim3(256), 0, stream, tiled, static_cast<int>(nb),
                       rows, rows_padded, a16, m, y, addend, addend_stride);
  else
    hipLaunchKernelGGL((gemm_rb_kernel<kTypeIq4Xs, MF, NF>), grid, dim3(256), 0, stream, tiled,
                       static_cast<int>(nb), rows, rows_padded, a16, m, y, addend, addend_stride);
}

uint64_t tiles(uint64_t rows, uint64_t m, uint64_t bn, uint64_t bm) {
  return ((rows + bn - 1) / bn) * ((m + bm - 1) / bm);
}

}  // namespace

int gemm_default_variant(uint64_t rows, uint64_t m) {
  // Register-B 128 x 128 tiles (two work-groups per CU fit, 2 waves per
  // SIMD); the 128 x 256 tile only once there are work-groups for every CU
  // several times over.
  if (tiles(rows, m, 256, 128) >= 1024) return 2;
  return 3;
}

void launch_gemm(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, const uint16_t* a16, uint64_t m,
                 float* y, const float* addend, uint64_t addend_stride, int variant, hipStream_t stream) {
  if (variant == 0) variant = gemm_default_variant(rows, m);
  switch (variant) {
    case 2:
      launch_gemm_rb<8, 4>(type, tiled, rows, nb, a16, m, y, addend, addend_stride, stream);
      return;
    case 3:
      launch_gemm_rb<8, 2>(type, tiled, rows, nb, a16, m, y, addend, addend_stride, stream);
      return;
    case 4:
      launch_gemm_rb<4, 4>(type, tiled, rows, nb, a16, m, y, addend, addend_stride, stream);
      return;
    default:
      break;
  }
  const uint64_t rows_padded = (rows + 7) / 8 * 8;
  dim3 grid(static_cast<unsigned>((rows + kBN - 1) / kBN), static_cast<unsigned>((m + kBM - 1) / kBM));
  if (type == kTypeQ4K)
    hipLaunchKernelGGL(gemm_kernel<kTypeQ4K>, grid, dim3(256), 0, stream, tiled, static_cast<int>(nb), rows,
                       rows_padded, a16, m, y, addend, addend_stride);
  else
    hipLaunchKernelGGL(gemm_kernel<kTypeIq4Xs>, grid, dim3(256), 0, stream, tiled, static_cast<int>(nb), rows,
                       rows_padded, a16, m, y, addend, addend_stride);
}

}  // namespace mq
