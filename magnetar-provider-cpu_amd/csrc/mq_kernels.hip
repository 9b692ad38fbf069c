// gfx950 kernels for the GGUF block-quantized matmul path: tile repack,
// bit-exact dequantization, int8 activation quantization, the decode GEMV
// and the MFMA prefill GEMM.
//
// Built with -ffp-contract=off: no multiply-add is fused unless written as
// fmaf, so the dequantizer reproduces the reference's separately rounded
// product and difference.
#include <cmath>
#include <type_traits>

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

// Lane exchanges inside each aligned group of 8 lanes by DPP (no LDS
// permute, no wait): quad_perm [1, 0, 3, 2] pairs lanes i ^ 1, quad_perm
// [2, 3, 0, 1] lanes i ^ 2, and row_half_mirror (i <-> 7 - i) pairs every
// lane with one of the other quad. Every lane of the group must be active.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141;

template <int CTRL>
__device__ inline int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

template <int CTRL>
__device__ inline float dpp_f32(float v) {
  return __int_as_float(dpp_i32<CTRL>(__float_as_int(v)));
}

// Four values of one 32-value block; the block's 8 lanes are consecutive,
// start at a multiple of 8, and all execute this together.
struct Quant4 {
  int q0, q1, q2, q3;
  float d;
  int half_sum;  // sum of q over this lane's 16-value half
  int run_sum;   // sum of q over the 32 values
};

__device__ inline Quant4 quantize4(float4 v) {
  Quant4 r;
  float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  // the max over the 8 lanes (fmaxf ignores NaN, in any order)
  amax = fmaxf(amax, dpp_f32<kDppXor1>(amax));
  amax = fmaxf(amax, dpp_f32<kDppXor2>(amax));
  amax = fmaxf(amax, dpp_f32<kDppHalfMirror>(amax));
  amax = fmaxf(0.0f, amax);
  r.d = amax / 127.0f;
  r.q0 = r.q1 = r.q2 = r.q3 = 0;
  if (amax != 0.0f) {
    r.q0 = sat_i8(rintf(v.x / r.d));
    r.q1 = sat_i8(rintf(v.y / r.d));
    r.q2 = sat_i8(rintf(v.z / r.d));
    r.q3 = sat_i8(rintf(v.w / r.d));
  }
  int hs = r.q0 + r.q1 + r.q2 + r.q3;
  hs += dpp_i32<kDppXor1>(hs);
  hs += dpp_i32<kDppXor2>(hs);
  r.half_sum = hs;  // the quad's 16 values
  r.run_sum = hs + dpp_i32<kDppHalfMirror>(hs);
  return r;
}

__device__ inline uint32_t pack_q4(const Quant4& q) {
  return (static_cast<uint32_t>(q.q0) & 0xFFu) | ((static_cast<uint32_t>(q.q1) & 0xFFu) << 8) |
         ((static_cast<uint32_t>(q.q2) & 0xFFu) << 16) | (static_cast<uint32_t>(q.q3) << 24);
}

__global__ void quantize_act_kernel(const float* __restrict__ x, uint64_t total,
                                    int8_t* __restrict__ values, float* __restrict__ scales,
                                    int32_t* __restrict__ sums) {
  uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  bool active = t < total / 4;
  float4 v = active ? reinterpret_cast<const float4*>(x)[t] : make_float4(0.f, 0.f, 0.f, 0.f);
  const Quant4 q = quantize4(v);
  if (!active) return;
  if (values) reinterpret_cast<uint32_t*>(values)[t] = pack_q4(q);
  int sub = static_cast<int>(t & 7);
  uint64_t blk = t >> 3;
  if (scales && sub == 0) scales[blk] = q.d;
  if (sums && (sub & 3) == 0) sums[2 * blk + (sub >> 2)] = q.half_sum;
}

// The f16 range of the prefill operands. f16 holds magnitudes up to 65504
// and has full precision only above 2^-14: unscaled, a row of large
// activations would turn into infinities and a row of tiny ones into
// subnormals. A power of two 2^e moves the largest magnitude into
// [2^14, 2^15): multiplying by it is exact in f32, and f16(v 2^e) =
// f16(v) 2^e wherever f16(v) is a normal number, so only the lost range is
// changed. Zero rows, and rows whose largest magnitude is infinite, keep
// e = 0. e stays within [-80, 80] (rows whose largest magnitude lies in
// [2^-65, 2^95]): with the weight's factor 2^f, f in [-40, 40], the
// output factor 2^-(e + f) is a normal f32.
__device__ inline int f16_range_exponent(float amax) {
  if (!(amax > 0.0f) || amax == __builtin_huge_valf()) return 0;
  const int ex = __builtin_amdgcn_frexp_expf(amax);  // amax = mantissa 2^ex, mantissa in [0.5, 1)
  const int e = 15 - ex;
  return e < -80 ? -80 : (e > 80 ? 80 : e);
}

// The output factor 2^-(e_r + f) of activation row `row` (clamped into the
// matrix). Each GEMM work-group loads its tile's factors in its prologue,
// one per thread, and keeps them in LDS for the epilogue, so that the
// epilogue's stores wait for no global load.
__device__ inline float out_factor(const F16Range& rg, uint64_t row, uint64_t m_rows) {
  return rg.row[row < m_rows ? row : m_rows - 1] * rg.down;
}

// One work-group per activation row: the row's largest magnitude (NaN
// ignored), then a16 = f16(v 2^e) with v = x, or the int8 round trip q d of
// x (quantize_act_kernel's blocks: lanes 8j .. 8j + 7 of a wave hold one
// 32-value block, since k % 32 == 0), and row_factor = 2^-e. HELD > 0: the
// row is at most 256 HELD float4, all loaded at once (indices clamped into
// the row, so no load waits behind a branch) and kept in registers between
// the two passes; HELD == 0: longer rows, read twice.
__device__ inline void store_f16x4(uint2* out, int t, float4 v, float up, int int8) {
  float f0 = v.x, f1 = v.y, f2 = v.z, f3 = v.w;
  if (int8) {
    const Quant4 q = quantize4(v);
    f0 = static_cast<float>(q.q0) * q.d;
    f1 = static_cast<float>(q.q1) * q.d;
    f2 = static_cast<float>(q.q2) * q.d;
    f3 = static_cast<float>(q.q3) * q.d;
  }
  __half2 h01 = __floats2half2_rn(f0 * up, f1 * up), h23 = __floats2half2_rn(f2 * up, f3 * up);
  uint2 w;
  w.x = *reinterpret_cast<uint32_t*>(&h01);
  w.y = *reinterpret_cast<uint32_t*>(&h23);
  out[t] = w;
}

__device__ inline float absmax4(float4 v) {
  return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}

template <int HELD>
__global__ __launch_bounds__(256) void activations_f16_kernel(const float* __restrict__ x, uint64_t k, int int8,
                                                              uint16_t* __restrict__ a16,
                                                              float* __restrict__ row_factor) {
  const uint64_t row = blockIdx.x;
  const float4* xr = reinterpret_cast<const float4*>(x + row * k);
  uint2* out = reinterpret_cast<uint2*>(a16 + row * k);
  const int n4 = static_cast<int>(k / 4);
  const int tid = static_cast<int>(threadIdx.x);
  float4 v[HELD > 0 ? HELD : 1];
  float amax = 0.0f;
  if constexpr (HELD > 0) {
#pragma unroll
    for (int i = 0; i < HELD; ++i) v[i] = xr[min(tid + 256 * i, n4 - 1)];
#pragma unroll
    for (int i = 0; i < HELD; ++i)
      if (tid + 256 * i < n4) amax = fmaxf(amax, absmax4(v[i]));
  } else {
    for (int t = tid; t < n4; t += 256) amax = fmaxf(amax, absmax4(xr[t]));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  __shared__ float wave_max[4];
  if ((tid & 63) == 0) wave_max[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3]));
  const int e = f16_range_exponent(amax);
  const float up = __builtin_amdgcn_ldexpf(1.0f, e);
  if (tid == 0) row_factor[row] = __builtin_amdgcn_ldexpf(1.0f, -e);
  // a 32-value block's 8 lanes are all in the row or all past it (n4 % 8
  // == 0), so the quantization's lane exchanges stay among active lanes
  if constexpr (HELD > 0) {
#pragma unroll
    for (int i = 0; i < HELD; ++i) {
      const int t = tid + 256 * i;
      if (t < n4) store_f16x4(out, t, v[i], up, int8);
    }
  } else {
    for (int t = tid; t < n4; t += 256) store_f16x4(out, t, xr[t], up, int8);
  }
}

// out = max |x| as f32 bits (non-negative floats order as their bits): one
// atomic per work-group, float4 reads (n % 4 == 0).
__global__ __launch_bounds__(256) void absmax_kernel(const float* __restrict__ x, uint64_t n,
                                                     uint32_t* __restrict__ out) {
  float amax = 0.0f;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n / 4; i += static_cast<uint64_t>(gridDim.x) * 256) {
    const float4 v = x4[i];
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  __shared__ float wave_max[4];
  if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = amax;
  __syncthreads();
  if (threadIdx.x == 0)
    atomicMax(out, __float_as_uint(fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3]))));
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

// Split-K epilogue across work-groups, deterministic: each work-group
// writes its (acc, mins) for its 64 rows to partials[ks], then takes a
// ticket on its row block's counter; the work-group that takes the last
// ticket adds the KS partials in ks order, writes y and resets the counter
// to zero for the next call. No work-group waits on another.
//
// Visibility without an L2 flush: the partials are written and read with
// relaxed agent-scope atomic stores/loads (global_store/load ... sc1, which
// are coherent across the XCDs' L2s), and the stores are waited on
// (s_waitcnt vmcnt(0)) before the ticket is taken, so every partial is at
// the coherence point before its work-group's ticket. A release/acquire
// fence at agent scope would do the same for plain stores, but costs a
// write-back and an invalidation of the whole L2 (buffer_wbl2 / buffer_inv),
// which stalls every other work-group on the XCD.
constexpr int kWaitVmcnt0 = 0x0F70;  // s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15): stores only

// Decode-step fusions of the LDS-form GEMV (m = 1), fixed per launch:
//  NORM: the activation row is rmsnorm'd in the staging, x * scale * w with
//   scale = 1 / sqrt(mean(x^2) + eps) (src/lib.rs:348-402), before the int8
//   quantization;
//  kEpiRope: rows below rope_rows are rotated in interleaved pairs (rows
//   2i, 2i + 1 of a head of rope_dim) at `position` (src/lib.rs:616-687),
//   and rows are routed to three outputs by row range (Q, then the K and V
//   caches' rows: the kv-write, src/lib.rs:740-768);
//  kEpiSiluPairs: the stored rows interleave gate and up by blocks of 32
//   (block 2i = gate rows 32i.., block 2i + 1 = up rows 32i..), and the
//   output is silu(gate) * up (src/lib.rs:2592-2596, 993-1004).
constexpr int kEpiPlain = 0, kEpiRope = 1, kEpiSiluPairs = 2;

using Fusion = GemvFusion;

__device__ inline float wave_sum64(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Work-group barrier that waits for this wave's LDS operations only (not
// for its vector-memory loads in flight, as __syncthreads() would).
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Thread t's share of the row's sum of squares: float4 elements t,
// t + blockDim, ... in that order.
__device__ inline void add_squares(float& ss, float4 a) {
  ss += a.x * a.x;
  ss += a.y * a.y;
  ss += a.z * a.z;
  ss += a.w * a.w;
}

// 1 / sqrt(mean(x^2) + eps) from the threads' shares, over the work-group.
__device__ inline float norm_from_squares(float ss, uint64_t K, float eps) {
  __shared__ float part[8];
  ss = wave_sum64(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float total = 0.0f;
  for (int i = 0; i < static_cast<int>(blockDim.x >> 6); ++i) total += part[i];
  return 1.0f / sqrtf(total / static_cast<float>(K) + eps);
}

// norm_from_squares when thread t holds float4 element t of the row and
// nothing else (K / 4 == blockDim.x, the one-super-block-per-wave GEMV):
// the same elements, order and value, behind a barrier that waits for LDS
// only, so the weight loads already in flight are not waited for.
__device__ inline float wave_norm_scale(float4 v, uint64_t K, float eps) {
  __shared__ __attribute__((aligned(16))) float part[16];
  float ss = 0.0f;
  add_squares(ss, v);
  ss = wave_sum64(ss);
  const int S = static_cast<int>(blockDim.x >> 6);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  if (static_cast<int>(threadIdx.x) < 16 - S) part[S + threadIdx.x] = 0.0f;  // adds nothing below
  lds_barrier();
  // the waves' sums in wave order, read four at a time
  float total = 0.0f;
  const float4* p4 = reinterpret_cast<const float4*>(part);
  for (int i = 0; i < (S + 3) / 4; ++i) {
    const float4 q = p4[i];
    total += q.x;
    total += q.y;
    total += q.z;
    total += q.w;
  }
  return 1.0f / sqrtf(total / static_cast<float>(K) + eps);
}

// 1 / sqrt(mean(x^2) + eps) of the activation row, over the work-group
// (the whole row, whatever the work-group's K range).
__device__ inline float row_norm_scale(const float* __restrict__ x, uint64_t K, float eps) {
  float ss = 0.0f;
  for (uint64_t i = threadIdx.x; i < K / 4; i += blockDim.x) add_squares(ss, reinterpret_cast<const float4*>(x)[i]);
  return norm_from_squares(ss, K, eps);
}

// Stores one lane's row results (every lane of the wave calls it: the
// epilogues exchange values across lanes).
template <int M, int EPI>
__device__ inline void store_out(const float (&v)[M], uint64_t row, bool valid, int lane, uint64_t rows, float* y,
                                 const Fusion& fu) {
  if constexpr (EPI == kEpiPlain) {
    if (valid) {
#pragma unroll
      for (int m = 0; m < M; ++m) y[m * rows + row] = v[m];
    }
  } else if constexpr (EPI == kEpiRope) {
    static_assert(M == 1, "decode-step epilogues take one activation row");
    const float other = __shfl_xor(v[0], 1);
    float o = v[0];
    if (row < fu.rope_rows) {
      const uint32_t p = static_cast<uint32_t>(row % fu.rope_dim) / 2;
      const float angle = fu.position * fu.freq[p];
      const float sn = sinf(angle), cs = cosf(angle);
      // pair (a, b) = (even row, odd row): a c - b s, a s + b c
      o = (lane & 1) == 0 ? v[0] * cs - other * sn : other * sn + v[0] * cs;
    }
    if (valid) {
      const int seg = row >= fu.seg_begin[2] ? 2 : row >= fu.seg_begin[1] ? 1 : 0;
      fu.seg_out[seg][row - fu.seg_begin[seg]] = o;
    }
  } else {
    static_assert(M == 1, "decode-step epilogues take one activation row");
    const float u = __shfl_down(v[0], 32);
    if (lane < 32 && valid) {
      const float g = v[0];
      const float sg = g * (1.0f / (1.0f + expf(-g)));
      y[(row - lane) / 2 + lane] = sg * u;
    }
  }
}

template <int M, int EPI>
__device__ inline void splitk_finish(float (&acc)[M], float (&mins)[M], uint64_t rows, float* y,
                                     const float* addend, uint64_t addend_stride, float* partials,
                                     uint32_t* counters, int KS, const Fusion& fu) {
  const int lane = threadIdx.x & 63;
  const uint64_t rb = blockIdx.x, ks = blockIdx.y;
  const uint64_t rows64 = static_cast<uint64_t>(gridDim.x) * 64;
  const uint64_t row = rb * 64 + lane;
  // layout: partials[ks][m][2][rows64]
#pragma unroll
  for (int m = 0; m < M; ++m) {
    __hip_atomic_store(&partials[((ks * M + m) * 2 + 0) * rows64 + row], acc[m], __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&partials[((ks * M + m) * 2 + 1) * rows64 + row], mins[m], __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  // The relaxed stores, the wait and the relaxed ticket are ordered for the
  // hardware by the wait alone; the signal fences keep the compiler from
  // moving any of these memory operations across it (a fence of no scope
  // beyond the thread emits no instruction).
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  uint32_t ticket = 0;
  if (lane == 0) ticket = __hip_atomic_fetch_add(&counters[rb], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  ticket = __shfl(ticket, 0);
  if (ticket != static_cast<uint32_t>(KS - 1)) return;
  // the partial loads below stay after the ticket that admits them
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  const bool valid = row < rows;
  float v[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float a = 0.0f, mn = 0.0f;
    for (int i = 0; i < KS; ++i) {
      a += __hip_atomic_load(&partials[((i * M + m) * 2 + 0) * rows64 + row], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      mn += __hip_atomic_load(&partials[((i * M + m) * 2 + 1) * rows64 + row], __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
    }
    v[m] = a - mn;
    if (addend && valid) v[m] = v[m] + addend[m * addend_stride + row];
  }
  store_out<M, EPI>(v, row, valid, lane, rows, y, fu);
  if (lane == 0) __hip_atomic_store(&counters[rb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cross-wave (within a work-group) reduction through the kernel's dynamic
// LDS, then either the store of y (KS == 1) or the split-K epilogue.
template <int M, int EPI = kEpiPlain>
__device__ inline void finish_rows(float (&acc)[M], float (&mins)[M], uint64_t rows, float* y, const float* addend,
                                   uint64_t addend_stride, float* red, float* partials, uint32_t* counters, int KS,
                                   const Fusion& fu = Fusion{}) {
  const int lane = threadIdx.x & 63, s = threadIdx.x >> 6, S = blockDim.x >> 6;
  if (M == 1 && KS == 1 && S > 1) {
    // one activation row: each wave hands over acc - mins, so wave 0 sums
    // S values per row (in wave order) rather than 2 S
    __syncthreads();  // every wave is done reading activations
    red[s * 64 + lane] = acc[0] - mins[0];
    __syncthreads();
    if (s != 0) return;
    float v = red[lane];
    for (int i = 1; i < S; ++i) v += red[i * 64 + lane];
    acc[0] = v;
    mins[0] = 0.0f;
  } else if (S > 1) {
    __syncthreads();  // every wave is done reading activations
#pragma unroll
    for (int m = 0; m < M; ++m) {
      red[((s * M + m) * 2 + 0) * 64 + lane] = acc[m];
      red[((s * M + m) * 2 + 1) * 64 + lane] = mins[m];
    }
    __syncthreads();
    if constexpr (M > 1 && EPI == kEpiPlain) {
      if (KS == 1 && S >= M) {
        // one wave per activation row: wave s sums row s's partials in
        // wave order (the same order and values as below) and stores it
        if (s >= M) return;
        float a = red[(s * 2 + 0) * 64 + lane], mn = red[(s * 2 + 1) * 64 + lane];
        for (int i = 1; i < S; ++i) {
          a += red[((i * M + s) * 2 + 0) * 64 + lane];
          mn += red[((i * M + s) * 2 + 1) * 64 + lane];
        }
        const uint64_t row = static_cast<uint64_t>(blockIdx.x) * 64 + lane;
        if (row < rows) {
          float v = a - mn;
          if (addend) v = v + addend[s * addend_stride + row];
          y[s * rows + row] = v;
        }
        return;
      }
    }
    if (s != 0) return;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float a = red[(m * 2 + 0) * 64 + lane], mn = red[(m * 2 + 1) * 64 + lane];
      for (int i = 1; i < S; ++i) {
        a += red[((i * M + m) * 2 + 0) * 64 + lane];
        mn += red[((i * M + m) * 2 + 1) * 64 + lane];
      }
      acc[m] = a;
      mins[m] = mn;
    }
  }
  if (KS > 1) {
    splitk_finish<M, EPI>(acc, mins, rows, y, addend, addend_stride, partials, counters, KS, fu);
    return;
  }
  const uint64_t row = static_cast<uint64_t>(blockIdx.x) * 64 + lane;
  const bool valid = row < rows;
  float v[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    v[m] = acc[m] - mins[m];
    if (addend && valid) v[m] = v[m] + addend[m * addend_stride + row];
  }
  store_out<M, EPI>(v, row, valid, lane, rows, y, fu);
}

// ---------------------------------------------------------------------------
// Activation staging of the LDS form. Staging is split in two phases so the
// work-group's activation loads are issued before its weight loads: vector
// memory returns in issue order per wave, and the staging barrier would
// otherwise wait behind the first weight blocks. Phase 1 (load) issues the
// first kPre per-thread loads into registers; phase 2 (store) writes them
// to LDS, then loads and writes whatever the registers did not cover.
//
// LDS layout of the K range [k0, k0 + kn) for m rows: int8 values [m][kn],
// then per run f32 pairs (d, d * (s0 + s1)) for Q4_K, or f32 d for IQ4_XS,
// indexed [m][kn / 32].
// ---------------------------------------------------------------------------

// Fused form: quantize the f32 activations straight into LDS with the same
// per-block arithmetic as quantize_act_kernel (bit-identical values, scales
// and sums). Every thread runs the same iterations so the 8-lane groups of
// quantize4 shuffle together. Only the first kv values of each row's range
// exist (kv < kn for a plane format whose K ends inside a group); the rest
// are staged as zeros with d = 0.
template <int TYPE, int M, bool NORM = false>
struct FusedStage {
  static constexpr int kPre = 4;
  float4 v[kPre];
  float4 g[NORM ? kPre : 1];  // NORM: the rmsnorm weight at the same positions (M == 1)

  __device__ void load(const float* __restrict__ xf, uint64_t K, uint64_t k0, int kn, int kv,
                       const float* __restrict__ nw = nullptr) {
    const int n4 = M * kn / 4, per_row4 = kn / 4;
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
      const int i = j * static_cast<int>(blockDim.x) + static_cast<int>(threadIdx.x);
      v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
      const int m = M == 1 ? 0 : i / per_row4, c4 = i - m * per_row4;
      if (i < n4 && 4 * c4 < kv) v[j] = *reinterpret_cast<const float4*>(xf + m * K + k0 + 4 * c4);
      if constexpr (NORM) {
        g[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < n4 && 4 * c4 < kv) g[j] = *reinterpret_cast<const float4*>(nw + k0 + 4 * c4);
      }
    }
  }

  // x * scale * w, each product rounded (the rmsnorm's order)
  __device__ static float4 normed(float4 x, float scale, float4 w) {
    return make_float4(x.x * scale * w.x, x.y * scale * w.y, x.z * scale * w.z, x.w * scale * w.w);
  }

  __device__ static void put(const Quant4& q, int i, uint8_t* lds, int M_kn) {
    float* rs = reinterpret_cast<float*>(lds + M_kn);
    reinterpret_cast<uint32_t*>(lds)[i] = pack_q4(q);
    const int run = i >> 3;  // m * (kn / 32) + run within the range
    if (is_plane_format(TYPE)) {
      // record (d, half sum 0, half sum 1, 0) per run
      uint32_t* rec = reinterpret_cast<uint32_t*>(rs) + 4 * run;
      if ((i & 7) == 0) {
        rec[0] = __float_as_uint(q.d);
        rec[1] = static_cast<uint32_t>(q.half_sum);
      } else if ((i & 7) == 4) {
        rec[2] = static_cast<uint32_t>(q.half_sum);
      }
    } else if ((i & 7) == 0) {
      if (TYPE == kTypeQ4K) {
        rs[2 * run] = q.d;
        rs[2 * run + 1] = q.d * static_cast<float>(q.run_sum);
      } else {
        rs[run] = q.d;
      }
    }
  }

  // The rmsnorm scale of the (one) activation row. When the registers hold
  // the whole row (no K split, K / 4 <= kPre * blockDim) its squares add up
  // from them, the elements and order of row_norm_scale (the same value),
  // without reading x again behind the weight loads already issued.
  __device__ float norm_scale(const float* __restrict__ xf, uint64_t K, int kn, float eps) const {
    if (static_cast<uint64_t>(kn) != K || K / 4 > kPre * static_cast<uint64_t>(blockDim.x))
      return row_norm_scale(xf, K, eps);
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < kPre; ++j)
      if (static_cast<uint64_t>(j) * blockDim.x + threadIdx.x < K / 4) add_squares(ss, v[j]);
    return norm_from_squares(ss, K, eps);
  }

  __device__ void store(const float* __restrict__ xf, uint64_t K, uint64_t k0, int kn, int kv, uint8_t* lds,
                        float nscale = 1.0f, const float* __restrict__ nw = nullptr) const {
    const int n4 = M * kn / 4, per_row4 = kn / 4;
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
      const int i = j * static_cast<int>(blockDim.x) + static_cast<int>(threadIdx.x);
      float4 x = v[j];
      if constexpr (NORM) x = normed(x, nscale, g[j]);
      const Quant4 q = quantize4(x);
      if (i < n4) put(q, i, lds, M * kn);
    }
    for (int i0 = kPre * static_cast<int>(blockDim.x); i0 < n4; i0 += blockDim.x) {
      const int i = i0 + static_cast<int>(threadIdx.x);
      const bool act = i < n4;
      const int m = act ? i / per_row4 : 0, c4 = act ? i - m * per_row4 : 0;
      const bool in = act && 4 * c4 < kv;
      float4 x = in ? *reinterpret_cast<const float4*>(xf + m * K + k0 + 4 * c4) : make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (NORM) {
        const float4 w = in ? *reinterpret_cast<const float4*>(nw + k0 + 4 * c4) : make_float4(0.f, 0.f, 0.f, 0.f);
        x = normed(x, nscale, w);
      }
      const Quant4 q = quantize4(x);
      if (act) put(q, i, lds, M * kn);
    }
  }
};

// Pre-quantized activations: copy values and per-run scales (and Q4_K's
// d * (s0 + s1), or a plane format's half sums) into LDS.
template <int TYPE, int M>
struct QuantizedStage {
  static constexpr int kPre = 2;
  uint4 v[kPre];
  float d;
  int hs, hs1;

  __device__ void load(const int8_t* __restrict__ xv, const float* __restrict__ xs, const int32_t* __restrict__ xsum,
                       uint64_t K, uint64_t k0, int kn, int kv) {
    const int per_row16 = kn / 16, kruns = kn / 32;
    const int runs = static_cast<int>(K / 32), r0 = static_cast<int>(k0 / 32);
    const int t = static_cast<int>(threadIdx.x);
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
      const int i = j * static_cast<int>(blockDim.x) + t;
      v[j] = make_uint4(0, 0, 0, 0);
      const int m = M == 1 ? 0 : i / per_row16, c = i - m * per_row16;
      if (i < M * per_row16 && 16 * c < kv) v[j] = *reinterpret_cast<const uint4*>(xv + m * K + k0 + 16 * c);
    }
    d = 0.0f;
    hs = hs1 = 0;
    const int m = M == 1 ? 0 : t / kruns, u = t - m * kruns;
    if (t < M * kruns && 32 * u < kv) {
      const int src = m * runs + r0 + u;
      d = xs[src];
      if (TYPE == kTypeQ4K || is_plane_format(TYPE)) {
        const int2 sm = reinterpret_cast<const int2*>(xsum)[src];
        hs = TYPE == kTypeQ4K ? sm.x + sm.y : sm.x;
        hs1 = sm.y;
      }
    }
  }

  __device__ static void put_run(float* rs, int i, float d, int hs, int hs1) {
    if (is_plane_format(TYPE)) {
      reinterpret_cast<uint4*>(rs)[i] =
          make_uint4(__float_as_uint(d), static_cast<uint32_t>(hs), static_cast<uint32_t>(hs1), 0u);
    } else if (TYPE == kTypeQ4K) {
      rs[2 * i] = d;
      rs[2 * i + 1] = d * static_cast<float>(hs);
    } else {
      rs[i] = d;
    }
  }

  __device__ void store(const int8_t* __restrict__ xv, const float* __restrict__ xs, const int32_t* __restrict__ xsum,
                        uint64_t K, uint64_t k0, int kn, int kv, uint8_t* lds) const {
    const int per_row16 = kn / 16, kruns = kn / 32;
    const int runs = static_cast<int>(K / 32), r0 = static_cast<int>(k0 / 32);
    const int t = static_cast<int>(threadIdx.x);
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
      const int i = j * static_cast<int>(blockDim.x) + t;
      if (i < M * per_row16) reinterpret_cast<uint4*>(lds)[i] = v[j];
    }
    for (int i = kPre * static_cast<int>(blockDim.x) + t; i < M * per_row16; i += blockDim.x) {
      const int m = i / per_row16, c = i - m * per_row16;
      reinterpret_cast<uint4*>(lds)[i] =
          16 * c < kv ? *reinterpret_cast<const uint4*>(xv + m * K + k0 + 16 * c) : make_uint4(0, 0, 0, 0);
    }
    float* rs = reinterpret_cast<float*>(lds + M * kn);
    if (t < M * kruns) put_run(rs, t, d, hs, hs1);
    for (int i = static_cast<int>(blockDim.x) + t; i < M * kruns; i += blockDim.x) {
      const int m = i / kruns, u = i - m * kruns;
      const int src = m * runs + r0 + u;
      float dd = 0.0f;
      int h = 0, h1 = 0;
      if (32 * u < kv) {
        dd = xs[src];
        if (TYPE == kTypeQ4K || is_plane_format(TYPE)) {
          const int2 sm = reinterpret_cast<const int2*>(xsum)[src];
          h = TYPE == kTypeQ4K ? sm.x + sm.y : sm.x;
          h1 = sm.y;
        }
      }
      put_run(rs, i, dd, h, h1);
    }
  }
};

// ---------------------------------------------------------------------------
// Decode GEMV, row-per-lane with the activations staged in LDS (m <= 8).
// Grid: (row blocks of 64 stored rows) x KS K-splits. A work-group takes
// the super-blocks [b0, b1) of its split, its waves interleaved over them
// (wave s: b0 + s, b0 + s + S, ...). Each lane owns one stored row; a wave
// reads the row group tiles of its 8 row groups plane by plane (eight whole
// 128-byte lines per load).
//
// Schedule: activation loads, then the wave's first weight block, then the
// activations are written to LDS (or quantized there, FUSED) and the
// work-group synchronises once; each block's compute runs while the next
// block is loading. The weight loads are raw buffer loads predicated by
// offset, so every path issues the same loads and the waits stay exact.
//
// For m == 1 the LDS reads of chunk c + 1 (64 activation bytes and the
// chunk's two run scales) are issued before chunk c is computed, so the
// LDS latency is covered; with more rows the other rows' work covers it,
// and the reads happen at their use.
//
// Per run the integer dot is scaled by the 6-bit scale in integer
// arithmetic (exact), then by d_act in f32; d and dmin once per block.
// ---------------------------------------------------------------------------

struct SplitK {
  float* partials;
  uint32_t* counters;
  int ks;
};

// One super-block of one row as loaded: the header (Q4_K: 16 bytes; IQ4_XS:
// 8 bytes in .x/.y) and 8 planes of 16 quant bytes.
struct RawRowBlock {
  uint4 hdr;
  uint4 q[8];
};

// Loads one row's super-block from the work-group's weight resource:
// `offset` is the row group's tile of that block (kBufferNone: zeros, no
// access), `r` the row within the group.
template <int TYPE>
__device__ inline void load_row_block(RawRowBlock& a, __amdgpu_buffer_rsrc_t rsrc, uint32_t offset, int r) {
  if (TYPE == kTypeQ4K) {
    const uint32_t o = offset == kBufferNone ? kBufferNone : offset + r * 16;
    a.hdr = buffer_ld16(rsrc, o);
#pragma unroll
    for (int p = 0; p < 8; ++p) a.q[p] = buffer_ld16(rsrc, o == kBufferNone ? o : o + 128 * (p + 1));
  } else {
    const bool none = offset == kBufferNone;
    const uint2 h = buffer_ld8(rsrc, none ? kBufferNone : offset + r * 8);
    a.hdr = make_uint4(h.x, h.y, 0, 0);
#pragma unroll
    for (int p = 0; p < 8; ++p) a.q[p] = buffer_ld16(rsrc, none ? kBufferNone : offset + 64 + 128 * p + r * 16);
  }
}

// An LDS address the compiler cannot relate to its neighbours: the chunks'
// reads are adjacent in LDS, and without this the load-store vectorizer
// merges them across chunks and hoists every chunk's reads to the first,
// which only raises register pressure. The offsets are wave-uniform, so
// the read-first-lane changes no value.
__device__ inline const uint8_t* opaque(const uint8_t* base, int offset) {
  return base + __builtin_amdgcn_readfirstlane(offset);
}

// The activations of one chunk (64 values: Q4_K runs 2c and 2c + 1 are the
// low and high nibbles of 32 quant bytes; IQ4_XS runs 2c and 2c + 1 are 16
// quant bytes each) for M rows, as LDS broadcasts: 4 x 16 int8 and the two
// runs' scales (Q4_K: (d, d * sum) x 2; IQ4_XS: d x 2 in .x/.y).
template <int M>
struct Chunk {
  uint4 x[M][4];
  float4 s[M];
};

template <int TYPE, int M>
__device__ inline void read_chunk(Chunk<M>& ch, const uint8_t* lds, int kn, int kruns, int bl, int c) {
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const uint4* xa = reinterpret_cast<const uint4*>(opaque(lds, m * kn + bl * 256 + 64 * c));
    ch.x[m][0] = xa[0];
    ch.x[m][1] = xa[1];
    ch.x[m][2] = xa[2];
    ch.x[m][3] = xa[3];
    if (TYPE == kTypeQ4K) {
      ch.s[m] = reinterpret_cast<const float4*>(lds + M * kn)[m * (kruns / 2) + bl * 4 + c];
    } else {
      const float2 v = reinterpret_cast<const float2*>(lds + M * kn)[m * (kruns / 2) + bl * 4 + c];
      ch.s[m] = make_float4(v.x, v.y, 0.f, 0.f);
    }
  }
}

// Chunk c of one Q4_K row block: accumulates sc * dot * d_act into accb and
// m * d_act * sum into minb.
template <int M>
__device__ inline void q4k_chunk(const RawRowBlock& a, const Q4kSixBit& six, int c, const Chunk<M>& ch,
                                 float (&accb)[M], float (&minb)[M]) {
  int dlo[M], dhi[M];
#pragma unroll
  for (int m = 0; m < M; ++m) dlo[m] = dhi[m] = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint4 qq = a.q[2 * c + h];
    const uint32_t lo[4] = {qq.x & 0x0F0F0F0Fu, qq.y & 0x0F0F0F0Fu, qq.z & 0x0F0F0F0Fu, qq.w & 0x0F0F0F0Fu};
    const uint32_t hi[4] = {(qq.x >> 4) & 0x0F0F0F0Fu, (qq.y >> 4) & 0x0F0F0F0Fu, (qq.z >> 4) & 0x0F0F0F0Fu,
                            (qq.w >> 4) & 0x0F0F0F0Fu};
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4 x0 = ch.x[m][h], x1 = ch.x[m][2 + h];
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
    const float4 r = ch.s[m];
    accb[m] = fmaf(static_cast<float>(__mul24(dlo[m], static_cast<int>(sc0))), r.x, accb[m]);
    accb[m] = fmaf(static_cast<float>(__mul24(dhi[m], static_cast<int>(sc1))), r.z, accb[m]);
    minb[m] = fmaf(static_cast<float>(m0), r.y, minb[m]);
    minb[m] = fmaf(static_cast<float>(m1), r.w, minb[m]);
  }
}

// Chunk c of one IQ4_XS row block (runs 2c, 2c + 1): accumulates
// ls * dot * d_act into accb.
template <int M>
__device__ inline void iq4xs_chunk(const RawRowBlock& a, int c, const Chunk<M>& ch, float (&accb)[M]) {
  const uint2 hdr = make_uint2(a.hdr.x, a.hdr.y);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int j = 2 * c + h;
    const int ls = iq4xs_ls(hdr, j);
    const uint4 qq = a.q[j];
    const uint32_t lo[4] = {iq4_lookup4(qq.x & 0x0F0F0F0Fu), iq4_lookup4(qq.y & 0x0F0F0F0Fu),
                            iq4_lookup4(qq.z & 0x0F0F0F0Fu), iq4_lookup4(qq.w & 0x0F0F0F0Fu)};
    const uint32_t hi[4] = {iq4_lookup4((qq.x >> 4) & 0x0F0F0F0Fu), iq4_lookup4((qq.y >> 4) & 0x0F0F0F0Fu),
                            iq4_lookup4((qq.z >> 4) & 0x0F0F0F0Fu), iq4_lookup4((qq.w >> 4) & 0x0F0F0F0Fu)};
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4 x0 = ch.x[m][2 * h], x1 = ch.x[m][2 * h + 1];
      int dot = sdot4(lo[0], x0.x, 0);
      dot = sdot4(lo[1], x0.y, dot);
      dot = sdot4(lo[2], x0.z, dot);
      dot = sdot4(lo[3], x0.w, dot);
      dot = sdot4(hi[0], x1.x, dot);
      dot = sdot4(hi[1], x1.y, dot);
      dot = sdot4(hi[2], x1.z, dot);
      dot = sdot4(hi[3], x1.w, dot);
      accb[m] = fmaf(static_cast<float>(__mul24(dot, ls)), h == 0 ? ch.s[m].x : ch.s[m].y, accb[m]);
    }
  }
}

// The same chunks with the activations read from LDS at their use (for
// m >= 2, where holding a whole chunk per row would spill registers).
template <int M>
__device__ inline void q4k_chunk_direct(const RawRowBlock& a, const Q4kSixBit& six, int c, const uint8_t* lds,
                                        int kn, int kruns, int bl, float (&accb)[M], float (&minb)[M]) {
  int dlo[M], dhi[M];
#pragma unroll
  for (int m = 0; m < M; ++m) dlo[m] = dhi[m] = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint4 qq = a.q[2 * c + h];
    const uint32_t lo[4] = {qq.x & 0x0F0F0F0Fu, qq.y & 0x0F0F0F0Fu, qq.z & 0x0F0F0F0Fu, qq.w & 0x0F0F0F0Fu};
    const uint32_t hi[4] = {(qq.x >> 4) & 0x0F0F0F0Fu, (qq.y >> 4) & 0x0F0F0F0Fu, (qq.z >> 4) & 0x0F0F0F0Fu,
                            (qq.w >> 4) & 0x0F0F0F0Fu};
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4* xa = reinterpret_cast<const uint4*>(opaque(lds, m * kn + bl * 256 + 64 * c + 16 * h));
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
    const float4 r = reinterpret_cast<const float4*>(lds + M * kn)[m * (kruns / 2) + bl * 4 + c];
    accb[m] = fmaf(static_cast<float>(__mul24(dlo[m], static_cast<int>(sc0))), r.x, accb[m]);
    accb[m] = fmaf(static_cast<float>(__mul24(dhi[m], static_cast<int>(sc1))), r.z, accb[m]);
    minb[m] = fmaf(static_cast<float>(m0), r.y, minb[m]);
    minb[m] = fmaf(static_cast<float>(m1), r.w, minb[m]);
  }
}

template <int M>
__device__ inline void iq4xs_chunk_direct(const RawRowBlock& a, int c, const uint8_t* lds, int kn, int kruns, int bl,
                                          float (&accb)[M]) {
  const uint2 hdr = make_uint2(a.hdr.x, a.hdr.y);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int j = 2 * c + h;
    const int ls = iq4xs_ls(hdr, j);
    const uint4 qq = a.q[j];
    const uint32_t lo[4] = {iq4_lookup4(qq.x & 0x0F0F0F0Fu), iq4_lookup4(qq.y & 0x0F0F0F0Fu),
                            iq4_lookup4(qq.z & 0x0F0F0F0Fu), iq4_lookup4(qq.w & 0x0F0F0F0Fu)};
    const uint32_t hi[4] = {iq4_lookup4((qq.x >> 4) & 0x0F0F0F0Fu), iq4_lookup4((qq.y >> 4) & 0x0F0F0F0Fu),
                            iq4_lookup4((qq.z >> 4) & 0x0F0F0F0Fu), iq4_lookup4((qq.w >> 4) & 0x0F0F0F0Fu)};
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4* xa = reinterpret_cast<const uint4*>(opaque(lds, m * kn + bl * 256 + 32 * j));
      const uint4 x0 = xa[0], x1 = xa[1];
      int dot = sdot4(lo[0], x0.x, 0);
      dot = sdot4(lo[1], x0.y, dot);
      dot = sdot4(lo[2], x0.z, dot);
      dot = sdot4(lo[3], x0.w, dot);
      dot = sdot4(hi[0], x1.x, dot);
      dot = sdot4(hi[1], x1.y, dot);
      dot = sdot4(hi[2], x1.z, dot);
      dot = sdot4(hi[3], x1.w, dot);
      accb[m] = fmaf(static_cast<float>(__mul24(dot, ls)), reinterpret_cast<const float*>(lds + M * kn)[m * kruns + bl * 8 + j],
                     accb[m]);
    }
  }
}

// One row block through all 4 chunks. With PIPE, `next` holds chunk 0 of
// this block on entry and chunk 0 of block bl_next (when has_next) on exit.
template <int TYPE, int M, bool PIPE>
__device__ inline void row_block(const RawRowBlock& a, const uint8_t* lds, int kn, int kruns, int bl, int bl_next,
                                 bool has_next, Chunk<M>& next, float (&acc)[M], float (&mins)[M]) {
  float accb[M], minb[M];
#pragma unroll
  for (int m = 0; m < M; ++m) accb[m] = minb[m] = 0.0f;
  Q4kSixBit six;
  if (TYPE == kTypeQ4K) six = q4k_six_bit(a.hdr);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    if (PIPE) {
      const Chunk<M> cur = next;
      if (c < 3)
        read_chunk<TYPE, M>(next, lds, kn, kruns, bl, c + 1);
      else if (has_next)
        read_chunk<TYPE, M>(next, lds, kn, kruns, bl_next, 0);
      if (TYPE == kTypeQ4K)
        q4k_chunk<M>(a, six, c, cur, accb, minb);
      else
        iq4xs_chunk<M>(a, c, cur, accb);
    } else if (TYPE == kTypeQ4K) {
      q4k_chunk_direct<M>(a, six, c, lds, kn, kruns, bl, accb, minb);
    } else {
      iq4xs_chunk_direct<M>(a, c, lds, kn, kruns, bl, accb);
    }
  }
  if (TYPE == kTypeQ4K) {
    const float d = half_bits(a.hdr.x), dmin = half_bits(a.hdr.x >> 16);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      acc[m] = fmaf(d, accb[m], acc[m]);
      mins[m] = fmaf(dmin, minb[m], mins[m]);
    }
  } else {
    const float d = half_bits(a.hdr.x);
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = fmaf(d, accb[m], acc[m]);
  }
}

// Wave-local staging of two super-blocks bA and bB (bB past b1 is skipped)
// of the K range that starts at block b0: the wave that multiplies them
// stages their activations into their LDS slots itself, so no work-group
// barrier orders staging before math. load() issues the global reads (before
// the wave's weight blocks: per-wave returns come in issue order), put()
// writes LDS. Fused: quantize4 of each block's 256 f32 values, the
// arithmetic of the work-group staging (bit-identical). Pre-quantized: lanes
// 0..31 copy the two blocks' int8 values (16 B each), lanes 32..47 their
// runs' scales (and sums), through buffer loads predicated by offset (no
// branch for a merge to wait on).
__device__ inline float4 u4_as_f4(uint4 v) {
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

template <int TYPE, int M, bool FUSED, bool TWO = true>
struct WaveStage {
  float4 xa[M], xb[M];
  uint4 vv[M];
  uint32_t dd[M];
  uint2 hh[M];

  __device__ void load(const float* __restrict__ xf, const int8_t* __restrict__ xv, const float* __restrict__ xs,
                       const int32_t* __restrict__ xsum, uint64_t K, int bA, int bB, int b1, int lane) {
    if constexpr (FUSED) {
      // buffer loads predicated by offset (blocks past b1 read zeros): no
      // branch, so none of the weight loads that follow waits behind them
      const __amdgpu_buffer_rsrc_t rsx = buffer_rsrc(xf, static_cast<uint32_t>(M * K * 4));
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint32_t row = static_cast<uint32_t>(m * K * 4) + 16 * static_cast<uint32_t>(lane);
        xa[m] = u4_as_f4(buffer_ld16(rsx, bA < b1 ? row + 1024 * static_cast<uint32_t>(bA) : kBufferNone));
        if (TWO) xb[m] = u4_as_f4(buffer_ld16(rsx, bB < b1 ? row + 1024 * static_cast<uint32_t>(bB) : kBufferNone));
      }
    } else if constexpr (!TWO) {
      // one block: lane group g = lane / 16 copies the values of rows g,
      // g + 4 (16 B per lane), lane group lane / 8 the run data of row
      // lane / 8, so no lane holds more than two rows' worth
      const uint32_t runs = static_cast<uint32_t>(K / 32);
      const __amdgpu_buffer_rsrc_t rsv = buffer_rsrc(xv, static_cast<uint32_t>(M * K));
      const __amdgpu_buffer_rsrc_t rss = buffer_rsrc(xs, static_cast<uint32_t>(M * runs * 4));
      const __amdgpu_buffer_rsrc_t rsh = buffer_rsrc(xsum, TYPE == kTypeQ4K ? static_cast<uint32_t>(M * runs * 8) : 0u);
      const bool live = bA < b1;
#pragma unroll
      for (int i = 0; i < (M + 3) / 4; ++i) {
        const int m = (lane >> 4) + 4 * i;
        const uint32_t c16 = static_cast<uint32_t>(m * K + 256 * bA + 16 * (lane & 15));
        vv[i] = buffer_ld16(rsv, live && m < M ? c16 : kBufferNone);
      }
      const int mr = lane >> 3;
      const uint32_t src = static_cast<uint32_t>(mr) * runs + 8 * bA + (lane & 7);
      dd[0] = buffer_ld4(rss, live && mr < M ? 4 * src : kBufferNone);
      hh[0] = buffer_ld8(rsh, live && mr < M ? 8 * src : kBufferNone);
    } else {
      const uint32_t runs = static_cast<uint32_t>(K / 32);
      const __amdgpu_buffer_rsrc_t rsv = buffer_rsrc(xv, static_cast<uint32_t>(M * K));
      const __amdgpu_buffer_rsrc_t rss = buffer_rsrc(xs, static_cast<uint32_t>(M * runs * 4));
      const __amdgpu_buffer_rsrc_t rsh = buffer_rsrc(xsum, TYPE == kTypeQ4K ? static_cast<uint32_t>(M * runs * 8) : 0u);
      const bool is_val = lane < 32, is_run = lane >= 32 && lane < 48;
      const int blk = is_val ? (lane < 16 ? bA : bB) : (lane < 40 ? bA : bB);
      const bool live = blk < b1 && (is_val || is_run);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint32_t c16 = static_cast<uint32_t>(m * K + 256 * blk + 16 * (lane & 15));
        const uint32_t src = static_cast<uint32_t>(m) * runs + 8 * blk + (lane & 7);
        vv[m] = buffer_ld16(rsv, live && is_val ? c16 : kBufferNone);
        dd[m] = buffer_ld4(rss, live && is_run ? 4 * src : kBufferNone);
        hh[m] = buffer_ld8(rsh, live && is_run ? 8 * src : kBufferNone);
      }
    }
  }

  // one fused activation row, one block, rmsnorm'd first: x * scale * w
  // (each product rounded, the rmsnorm's order)
  __device__ void put_normed(uint8_t* lds, int kn, int b0, int bA, int b1, int lane, float nscale, float4 w) const {
    static_assert(FUSED && M == 1 && !TWO, "the normed staging takes one f32 row, one block per wave");
    const Quant4 qa = quantize4(FusedStage<TYPE, 1, true>::normed(xa[0], nscale, w));
    if (bA < b1) FusedStage<TYPE, 1, false>::put(qa, 64 * (bA - b0) + lane, lds, kn);
  }

  __device__ void put(uint8_t* lds, int kn, int kruns, int b0, int bA, int bB, int b1, int lane) const {
    if constexpr (FUSED) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const Quant4 qa = quantize4(xa[m]);
        if (bA < b1) FusedStage<TYPE, M, false>::put(qa, m * (kn / 4) + 64 * (bA - b0) + lane, lds, M * kn);
        if (TWO) {
          const Quant4 qb = quantize4(xb[m]);
          if (bB < b1) FusedStage<TYPE, M, false>::put(qb, m * (kn / 4) + 64 * (bB - b0) + lane, lds, M * kn);
        }
      }
    } else if constexpr (!TWO) {
      const bool live = bA < b1;
      float* rs = reinterpret_cast<float*>(lds + M * kn);
      // lanes without a row store to a spare 16 bytes past the staging
      // (unused until the cross-wave sums): a store under a branch would
      // let the compiler sink its load below the weight loads
      const int spare = (M * kn + M * kruns * (TYPE == kTypeQ4K ? 8 : 4)) / 16;
#pragma unroll
      for (int i = 0; i < (M + 3) / 4; ++i) {
        const int m = (lane >> 4) + 4 * i;
        const int at = live && m < M ? m * (kn / 16) + 16 * (bA - b0) + (lane & 15) : spare;
        reinterpret_cast<uint4*>(lds)[at] = vv[i];
      }
      const int mr = lane >> 3;
      if (live && mr < M)
        QuantizedStage<TYPE, M>::put_run(rs, mr * kruns + 8 * (bA - b0) + (lane & 7), __uint_as_float(dd[0]),
                                         static_cast<int>(hh[0].x + hh[0].y), static_cast<int>(hh[0].y));
    } else {
      const bool is_val = lane < 32, is_run = lane >= 32 && lane < 48;
      const int blk = is_val ? (lane < 16 ? bA : bB) : (lane < 40 ? bA : bB);
      const bool live = blk < b1 && (is_val || is_run);
      float* rs = reinterpret_cast<float*>(lds + M * kn);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        if (live && is_val) reinterpret_cast<uint4*>(lds)[m * (kn / 16) + 16 * (blk - b0) + (lane & 15)] = vv[m];
        if (live && is_run)
          QuantizedStage<TYPE, M>::put_run(rs, m * kruns + 8 * (blk - b0) + (lane & 7), __uint_as_float(dd[m]),
                                           static_cast<int>(hh[m].x + hh[m].y), static_cast<int>(hh[m].y));
      }
    }
  }
};

template <int TYPE, int M, bool FUSED, bool NORM = false, int EPI = kEpiPlain>
__global__ __launch_bounds__(512) void gemv_lds_int8_kernel(
    const uint8_t* __restrict__ w, int nb, uint64_t rows, const int8_t* __restrict__ xv,
    const float* __restrict__ xs, const int32_t* __restrict__ xsum, const float* __restrict__ xf,
    float* __restrict__ y, const float* __restrict__ addend, uint64_t addend_stride, SplitK sk, Fusion fu) {
  static_assert(!NORM || (FUSED && M == 1), "the rmsnorm staging takes one f32 activation row");
  constexpr bool PIPE = M == 1;
  constexpr int kTile = TYPE == kTypeQ4K ? kQ4kTileBytes : kIq4xsTileBytes;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = blockDim.x >> 6;
  // balanced partition of the super-blocks: every split gets >= 1 (ks <= nb)
  const int b0 = static_cast<int>(blockIdx.y * nb / sk.ks), b1 = static_cast<int>((blockIdx.y + 1) * nb / sk.ks);
  const int r = lane & 7;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  const uint64_t k0 = static_cast<uint64_t>(b0) * 256;
  const int kn = (b1 - b0) * 256, kruns = kn / 32;
  // The work-group's 8 row groups as one buffer resource: rows past the
  // matrix read as zeros (their results are not stored).
  const uint64_t groups = (rows + 7) / 8, group_bytes = static_cast<uint64_t>(nb) * kTile;
  const uint64_t g0 = static_cast<uint64_t>(blockIdx.x) * 8;
  const uint64_t span = (groups - g0 < 8 ? groups - g0 : 8) * group_bytes;
  const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(w + g0 * group_bytes, static_cast<uint32_t>(span));
  const uint32_t lane_off = static_cast<uint32_t>((lane >> 3) * group_bytes);
  auto block_off = [&](int b) { return b < b1 ? lane_off + static_cast<uint32_t>(b) * kTile : kBufferNone; };

  float acc[M], mins[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = mins[m] = 0.0f;
  Chunk<M> next;
  const int bA = b0 + s;
  bool done = false;
  if constexpr (!NORM && M <= 4) {
    // Wave-local staging (up to 4 activation rows, when every wave has at
    // most two blocks; the bound is work-group uniform): the wave starts on
    // its first block as soon as that block and its activations have
    // landed, and both of its weight blocks are in flight from the start.
    if (b1 - b0 <= 2 * S) {
      const int bB = bA + S;
      WaveStage<TYPE, M, FUSED> ws;
      ws.load(xf, xv, xs, xsum, K, bA, bB, b1, lane);
      RawRowBlock A0, A1;
      load_row_block<TYPE>(A0, rsrc, block_off(bA), r);
      load_row_block<TYPE>(A1, rsrc, block_off(bB), r);
      ws.put(lds, kn, kruns, b0, bA, bB, b1, lane);
      if (bA < b1) {
        if (PIPE) read_chunk<TYPE, M>(next, lds, kn, kruns, bA - b0, 0);
        row_block<TYPE, M, PIPE>(A0, lds, kn, kruns, bA - b0, bB - b0, bB < b1, next, acc, mins);
      }
      if (bB < b1) row_block<TYPE, M, PIPE>(A1, lds, kn, kruns, bB - b0, bB + S - b0, false, next, acc, mins);
      done = true;
    }
  }
  if (!done) {
    // 1. activation loads
    FusedStage<TYPE, M, NORM> fs;
    QuantizedStage<TYPE, M> qs;
    if (FUSED)
      fs.load(xf, K, k0, kn, kn, fu.norm_w);
    else
      qs.load(xv, xs, xsum, K, k0, kn, kn);
    // 2. the wave's first weight block
    RawRowBlock A;
    load_row_block<TYPE>(A, rsrc, block_off(bA), r);
    // 3. activations into LDS (rmsnorm'd first under NORM)
    float nscale = 1.0f;
    if constexpr (NORM) nscale = fs.norm_scale(xf, K, kn, fu.norm_eps);
    if (FUSED)
      fs.store(xf, K, k0, kn, kn, lds, nscale, fu.norm_w);
    else
      qs.store(xv, xs, xsum, K, k0, kn, kn, lds);
    __syncthreads();
    if (PIPE && bA < b1) read_chunk<TYPE, M>(next, lds, kn, kruns, bA - b0, 0);
    for (int b = bA; b < b1; b += S) {
      const RawRowBlock cur = A;
      load_row_block<TYPE>(A, rsrc, block_off(b + S), r);
      // with more rows the scheduler would sink the prefetch below the math
      if (!PIPE) __builtin_amdgcn_sched_barrier(0);
      row_block<TYPE, M, PIPE>(cur, lds, kn, kruns, b - b0, b + S - b0, b + S < b1, next, acc, mins);
    }
  }
  finish_rows<M, EPI>(acc, mins, rows, y, addend, addend_stride, reinterpret_cast<float*>(lds), sk.partials,
                      sk.counters, sk.ks, fu);
}

// ---------------------------------------------------------------------------
// Decode GEMV with one super-block per wave (Q4_K, IQ4_XS; m <= 8): the
// LDS form's work-group of 64 stored rows with as many waves as the row has
// super-blocks (up to 16, 1024 threads), wave s taking block s of every
// row. Each wave stages its own block's activations (wave-local, no
// barrier before the math), so a wave holds one block of weights (36
// registers) instead of two: four waves per SIMD hide the math of one
// wave behind the loads of the others, and the math left after the last
// weight bytes arrive is one block. The waves' sums meet in LDS in wave
// order (finish_rows), so results are deterministic; they differ from the
// two-blocks-per-wave form by rounding only. No K split.
// ---------------------------------------------------------------------------

// (The f32 activations and the rmsnorm weight come right after the weight
// and its shape, within the kernel arguments preloaded into SGPRs.)
template <int TYPE, int M, bool FUSED, int EPI = kEpiPlain, bool NORM = false>
__global__ __launch_bounds__(1024) void gemv_wave_int8_kernel(
    const uint8_t* __restrict__ w, int nb, uint64_t rows, const float* __restrict__ xf,
    const float* __restrict__ norm_w, const int8_t* __restrict__ xv, const float* __restrict__ xs,
    const int32_t* __restrict__ xsum, float* __restrict__ y, const float* __restrict__ addend,
    uint64_t addend_stride, Fusion fu) {
  static_assert(M <= 8, "wave-local staging holds at most 8 activation rows");
  static_assert(!NORM || (FUSED && M == 1), "the rmsnorm staging takes one f32 activation row");
  // each chunk's activations read one chunk ahead while the registers allow
  // it (m = 4: 83 VGPRs, 10.4-10.7 -> 9.9 us at 14336 x 4096; m = 8 would
  // need another 80)
  constexpr bool PIPE = M <= 4;
  constexpr int kTile = TYPE == kTypeQ4K ? kQ4kTileBytes : kIq4xsTileBytes;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // the wave's super-block
  const int r = lane & 7;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  const int kn = nb * 256, kruns = kn / 32;
  const uint64_t groups = (rows + 7) / 8, group_bytes = static_cast<uint64_t>(nb) * kTile;
  const uint64_t g0 = static_cast<uint64_t>(blockIdx.x) * 8;
  const uint64_t span = (groups - g0 < 8 ? groups - g0 : 8) * group_bytes;
  const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(w + g0 * group_bytes, static_cast<uint32_t>(span));
  const uint32_t off = static_cast<uint32_t>((lane >> 3) * group_bytes) + static_cast<uint32_t>(s) * kTile;

  float acc[M], mins[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = mins[m] = 0.0f;
  Chunk<M> next;
  // activation loads first (per-wave returns come in issue order), then
  // the weight block, then the staging
  WaveStage<TYPE, M, FUSED, false> ws;
  ws.load(xf, xv, xs, xsum, K, s, nb, nb, lane);
  float4 nw = make_float4(0.f, 0.f, 0.f, 0.f);  // NORM: the rmsnorm weight at this lane's positions
  if constexpr (NORM)
    nw = u4_as_f4(buffer_ld16(buffer_rsrc(norm_w, static_cast<uint32_t>(K * 4)),
                              1024 * static_cast<uint32_t>(s) + 16 * static_cast<uint32_t>(lane)));
  __builtin_amdgcn_sched_barrier(0);
  RawRowBlock A;
  load_row_block<TYPE>(A, rsrc, off, r);
  // the weight loads issue before any use of the activations: left free,
  // the scheduler hoists the quantization's first operations above them,
  // and the wait for the activation load then holds the weight loads back
  // by a memory round trip
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (NORM) {
    // eps, a kernel argument past the preloaded ones, as a scalar load here
    // (left to the compiler it became a vector load after the barrier,
    // whose wait then covered every weight load in flight)
    const uint32_t eps_bits = __builtin_amdgcn_readfirstlane(__float_as_uint(fu.norm_eps));
    asm volatile("" ::"s"(eps_bits));
    ws.put_normed(lds, kn, 0, s, nb, lane, wave_norm_scale(ws.xa[0], K, __uint_as_float(eps_bits)), nw);
  }
  else
    ws.put(lds, kn, kruns, 0, s, nb, nb, lane);
  if (PIPE) read_chunk<TYPE, M>(next, lds, kn, kruns, s, 0);
  row_block<TYPE, M, PIPE>(A, lds, kn, kruns, s, nb, false, next, acc, mins);
  finish_rows<M, EPI>(acc, mins, rows, y, addend, addend_stride, reinterpret_cast<float*>(lds), nullptr, nullptr, 1,
                      fu);
}

// ---------------------------------------------------------------------------
// Narrow form of the LDS-staged int8 GEMV (Q4_K, IQ4_XS) for long rows over
// few output rows, e.g. the FFN down projection 4096 x 14336: 16 rows per
// work-group instead of 64, so 4096 rows fill the 256 CUs with 256
// work-groups and need no K split, whose cross-work-group reduction (the
// partials' agent-scope stores, the ticket, the re-read) costs several
// microseconds of round trips to memory. Lane = (quarter c = lane >> 4, row
// group (lane >> 3) & 1, row lane & 7): the four quarters of a wave take
// the four 64-value chunks of one super-block, so each lane loads only its
// chunk's two planes and the row's header, and the quarters' activation
// reads fall in distinct LDS banks. Wave s takes blocks s, s + S, ...,
// kNarrowDepth of them in the math and the next kNarrowDepth in flight. The
// quarters' sums meet by lane shuffles, the waves' through LDS. Sums are
// formed per chunk (d * (scaled chunk dot)), so results agree with the
// wide form to rounding, not bit for bit.
// ---------------------------------------------------------------------------

constexpr int kNarrowRows = 16;
constexpr int kNarrowDepth = 2;  // measured at 4096 x 14336 IQ4_XS: depth 1 9.4 us, 2 8.7, 4 10.4, 8 12.1

struct NarrowChunk {
  uint4 hdr;     // Q4_K: d | dmin, 12 scale bytes; IQ4_XS: d | scales_h, scales_l in .x, .y
  uint4 qa, qb;  // this row's two 16-byte planes of the chunk
};

template <int TYPE>
__device__ inline void load_narrow(NarrowChunk& a, __amdgpu_buffer_rsrc_t rsrc, uint32_t hdr_off, uint32_t plane_off,
                                   bool live) {
  if (TYPE == kTypeQ4K) {
    a.hdr = buffer_ld16(rsrc, live ? hdr_off : kBufferNone);
  } else {
    const uint2 h = buffer_ld8(rsrc, live ? hdr_off : kBufferNone);
    a.hdr = make_uint4(h.x, h.y, 0, 0);
  }
  a.qa = buffer_ld16(rsrc, live ? plane_off : kBufferNone);
  a.qb = buffer_ld16(rsrc, live ? plane_off + 128 : kBufferNone);
}

// Chunk c (runs 2c, 2c + 1) of block bl of one row against the staged
// activations of M rows: acc += d * (sc * dot * d_act), mins += dmin * (m *
// d_act * sum) (Q4_K), acc += d * (ls * dot * d_act) (IQ4_XS).
template <int TYPE, int M>
__device__ inline void narrow_chunk(const NarrowChunk& a, int c, const uint8_t* lds, int kn, int kruns, int bl,
                                    float (&acc)[M], float (&mins)[M]) {
  const uint8_t* xb = opaque(lds, bl * 256) + 64 * c;
  uint32_t lo[2][4], hi[2][4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint4 qq = h ? a.qb : a.qa;
    const uint32_t w4[4] = {qq.x, qq.y, qq.z, qq.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      lo[h][t] = w4[t] & 0x0F0F0F0Fu;
      hi[h][t] = (w4[t] >> 4) & 0x0F0F0F0Fu;
      if (TYPE == kTypeIq4Xs) {
        lo[h][t] = iq4_lookup4(lo[h][t]);
        hi[h][t] = iq4_lookup4(hi[h][t]);
      }
    }
  }
  if constexpr (TYPE == kTypeQ4K) {
    // runs 2c (low nibbles of both planes) and 2c + 1 (high nibbles)
    const uint32_t sc_w = c < 2 ? (a.hdr.y & 0x3F3F3F3Fu) : ((a.hdr.w & 0x0F0F0F0Fu) | ((a.hdr.y >> 2) & 0x30303030u));
    const uint32_t m_w =
        c < 2 ? (a.hdr.z & 0x3F3F3F3Fu) : (((a.hdr.w >> 4) & 0x0F0F0F0Fu) | ((a.hdr.z >> 2) & 0x30303030u));
    const int sh = 16 * (c & 1);
    const int sc0 = static_cast<int>((sc_w >> sh) & 0xFFu), sc1 = static_cast<int>((sc_w >> (sh + 8)) & 0xFFu);
    const float m0 = static_cast<float>((m_w >> sh) & 0xFFu), m1 = static_cast<float>((m_w >> (sh + 8)) & 0xFFu);
    const float d = half_bits(a.hdr.x), dmin = half_bits(a.hdr.x >> 16);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4* x = reinterpret_cast<const uint4*>(xb + m * kn);
      const uint4 x0 = x[0], x1 = x[1], x2 = x[2], x3 = x[3];
      int dlo = sdot4(lo[0][0], x0.x, 0);
      dlo = sdot4(lo[0][1], x0.y, dlo);
      dlo = sdot4(lo[0][2], x0.z, dlo);
      dlo = sdot4(lo[0][3], x0.w, dlo);
      dlo = sdot4(lo[1][0], x1.x, dlo);
      dlo = sdot4(lo[1][1], x1.y, dlo);
      dlo = sdot4(lo[1][2], x1.z, dlo);
      dlo = sdot4(lo[1][3], x1.w, dlo);
      int dhi = sdot4(hi[0][0], x2.x, 0);
      dhi = sdot4(hi[0][1], x2.y, dhi);
      dhi = sdot4(hi[0][2], x2.z, dhi);
      dhi = sdot4(hi[0][3], x2.w, dhi);
      dhi = sdot4(hi[1][0], x3.x, dhi);
      dhi = sdot4(hi[1][1], x3.y, dhi);
      dhi = sdot4(hi[1][2], x3.z, dhi);
      dhi = sdot4(hi[1][3], x3.w, dhi);
      const float4 r = reinterpret_cast<const float4*>(lds + M * kn)[m * (kruns / 2) + bl * 4 + c];
      float accb = static_cast<float>(__mul24(dlo, sc0)) * r.x;
      accb = fmaf(static_cast<float>(__mul24(dhi, sc1)), r.z, accb);
      float minb = m0 * r.y;
      minb = fmaf(m1, r.w, minb);
      acc[m] = fmaf(d, accb, acc[m]);
      mins[m] = fmaf(dmin, minb, mins[m]);
    }
  } else {
    // runs 2c (plane qa: values 0..15 low nibbles, 16..31 high) and 2c + 1 (qb)
    const uint2 hdr = make_uint2(a.hdr.x, a.hdr.y);
    const int ls0 = iq4xs_ls(hdr, 2 * c), ls1 = iq4xs_ls(hdr, 2 * c + 1);
    const float d = half_bits(a.hdr.x);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4* x = reinterpret_cast<const uint4*>(xb + m * kn);
      const uint4 x0 = x[0], x1 = x[1], x2 = x[2], x3 = x[3];
      int d0 = sdot4(lo[0][0], x0.x, 0);
      d0 = sdot4(lo[0][1], x0.y, d0);
      d0 = sdot4(lo[0][2], x0.z, d0);
      d0 = sdot4(lo[0][3], x0.w, d0);
      d0 = sdot4(hi[0][0], x1.x, d0);
      d0 = sdot4(hi[0][1], x1.y, d0);
      d0 = sdot4(hi[0][2], x1.z, d0);
      d0 = sdot4(hi[0][3], x1.w, d0);
      int d1 = sdot4(lo[1][0], x2.x, 0);
      d1 = sdot4(lo[1][1], x2.y, d1);
      d1 = sdot4(lo[1][2], x2.z, d1);
      d1 = sdot4(lo[1][3], x2.w, d1);
      d1 = sdot4(hi[1][0], x3.x, d1);
      d1 = sdot4(hi[1][1], x3.y, d1);
      d1 = sdot4(hi[1][2], x3.z, d1);
      d1 = sdot4(hi[1][3], x3.w, d1);
      const float2 sv = reinterpret_cast<const float2*>(lds + M * kn)[m * (kruns / 2) + bl * 4 + c];
      float accb = static_cast<float>(__mul24(d0, ls0)) * sv.x;
      accb = fmaf(static_cast<float>(__mul24(d1, ls1)), sv.y, accb);
      acc[m] = fmaf(d, accb, acc[m]);
    }
  }
}

template <int TYPE, int M, bool FUSED, bool NORM = false, int EPI = kEpiPlain>
__global__ __launch_bounds__(512) void gemv_narrow_kernel(const uint8_t* __restrict__ w, int nb, uint64_t rows,
                                                          const int8_t* __restrict__ xv, const float* __restrict__ xs,
                                                          const int32_t* __restrict__ xsum,
                                                          const float* __restrict__ xf, float* __restrict__ y,
                                                          const float* __restrict__ addend, uint64_t addend_stride,
                                                          Fusion fu) {
  static_assert(!NORM || (FUSED && M == 1), "the rmsnorm staging takes one f32 activation row");
  static_assert(EPI != kEpiSiluPairs, "the silu pairs span 64-row blocks");
  constexpr int kTile = TYPE == kTypeQ4K ? kQ4kTileBytes : kIq4xsTileBytes;
  constexpr int D = kNarrowDepth;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = blockDim.x >> 6;
  const int r = lane & 7, c = lane >> 4;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  const int kn = nb * 256, kruns = kn / 32;
  // the work-group's 2 row groups as one buffer resource (a missing second
  // group reads as zeros; its results are not stored)
  const uint64_t groups = (rows + 7) / 8, group_bytes = static_cast<uint64_t>(nb) * kTile;
  const uint64_t g0 = static_cast<uint64_t>(blockIdx.x) * (kNarrowRows / 8);
  const uint64_t span = (groups - g0 < 2 ? groups - g0 : 2) * group_bytes;
  const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(w + g0 * group_bytes, static_cast<uint32_t>(span));
  const uint32_t lane_off = static_cast<uint32_t>(((lane >> 3) & 1) * group_bytes);
  const uint32_t hdr_in = lane_off + (TYPE == kTypeQ4K ? 16u * r : 8u * r);
  const uint32_t plane_in = lane_off + (TYPE == kTypeQ4K ? 128u : 64u) + 256u * c + 16u * r;

  // Wave s multiplies blocks s, s + S, ...: with at most two per wave (and
  // up to 4 activation rows) it stages their activations itself, with no
  // work-group barrier; otherwise the work-group stages all of K.
  constexpr bool kWaveFit = M <= 4 && !NORM;
  const bool wave_staged = kWaveFit && nb <= 2 * S;  // work-group uniform
  FusedStage<TYPE, M, NORM> fs;
  QuantizedStage<TYPE, M> qs;
  WaveStage<TYPE, kWaveFit ? M : 1, FUSED> ws;
  if (wave_staged) {
    if constexpr (kWaveFit) ws.load(xf, xv, xs, xsum, K, s, s + S, nb, lane);
  } else if (FUSED) {
    fs.load(xf, K, 0, kn, kn, fu.norm_w);
  } else {
    qs.load(xv, xs, xsum, K, 0, kn, kn);
  }
  NarrowChunk cur[D];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const int b = s + j * S;
    load_narrow<TYPE>(cur[j], rsrc, hdr_in + b * kTile, plane_in + b * kTile, b < nb);
  }
  if (wave_staged) {
    if constexpr (kWaveFit) ws.put(lds, kn, kruns, 0, s, s + S, nb, lane);
  } else {
    float nscale = 1.0f;  // rmsnorm'd first under NORM
    if constexpr (NORM) nscale = fs.norm_scale(xf, K, kn, fu.norm_eps);
    if (FUSED)
      fs.store(xf, K, 0, kn, kn, lds, nscale, fu.norm_w);
    else
      qs.store(xv, xs, xsum, K, 0, kn, kn, lds);
    __syncthreads();
  }

  float acc[M], mins[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = mins[m] = 0.0f;
  for (int base = s; base < nb; base += D * S) {
    NarrowChunk nxt[D];
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int b = base + (D + j) * S;
      load_narrow<TYPE>(nxt[j], rsrc, hdr_in + b * kTile, plane_in + b * kTile, b < nb);
    }
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int b = base + j * S;  // wave-uniform
      if (b < nb) narrow_chunk<TYPE, M>(cur[j], c, lds, kn, kruns, b, acc, mins);
    }
#pragma unroll
    for (int j = 0; j < D; ++j) cur[j] = nxt[j];
  }
  // the four quarters of each row (lanes l, l ^ 16, l ^ 32, l ^ 48), then the waves
#pragma unroll
  for (int m = 0; m < M; ++m) {
    acc[m] += __shfl_xor(acc[m], 16);
    acc[m] += __shfl_xor(acc[m], 32);
    mins[m] += __shfl_xor(mins[m], 16);
    mins[m] += __shfl_xor(mins[m], 32);
  }
  __syncthreads();  // every wave is done reading activations
  float* red = reinterpret_cast<float*>(lds);
  if (lane < kNarrowRows) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      red[((s * M + m) * 2 + 0) * kNarrowRows + lane] = acc[m];
      red[((s * M + m) * 2 + 1) * kNarrowRows + lane] = mins[m];
    }
  }
  __syncthreads();
  if (s != 0) return;
  // wave 0 stays whole for the epilogue's lane pairs; lanes 16..63 repeat
  // lanes 0..15 and store nothing
  const int i16 = lane & (kNarrowRows - 1);
  const uint64_t row = static_cast<uint64_t>(blockIdx.x) * kNarrowRows + i16;
  const bool valid = lane < kNarrowRows && row < rows;
  float v[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float a = red[(m * 2 + 0) * kNarrowRows + i16], mn = red[(m * 2 + 1) * kNarrowRows + i16];
    for (int i = 1; i < S; ++i) {
      a += red[((i * M + m) * 2 + 0) * kNarrowRows + i16];
      mn += red[((i * M + m) * 2 + 1) * kNarrowRows + i16];
    }
    v[m] = a - mn;
    if (addend && valid) v[m] = v[m] + addend[m * addend_stride + row];
  }
  store_out<M, EPI>(v, row, valid, lane, rows, y, fu);
}

// ---------------------------------------------------------------------------
// Plane formats (Q8_0, Q4_0, IQ4_NL, Q5_K, Q6_K; layout in mq_device.h).
// One group (256 values) of one row is kPlanes 16-byte planes; run j of the
// group decodes to 32 values q (as 8 words of 4 bytes), a scale and a min
// per 16-value half, as the reference's `decode` (src/native/quant.rs:
// 102-149, 180-195) produces them.
// ---------------------------------------------------------------------------

__device__ inline uint32_t word_of(const uint4& v, int t) { return t == 0 ? v.x : t == 1 ? v.y : t == 2 ? v.z : v.w; }

// Signed bytes from nibbles 0..15 standing for nibble - 8 (Q4_0).
__device__ inline uint32_t nibbles_minus_8(uint32_t nib) {
  const uint32_t x = nib ^ 0x08080808u;
  return x | ((x & 0x08080808u) * 0x1Eu);  // bytes 0..7 stay, 8..15 gain 0xF0
}

// Signed bytes from 6-bit values 0..63 standing for value - 32 (Q6_K).
__device__ inline uint32_t six_bits_minus_32(uint32_t t) {
  const uint32_t x = t ^ 0x20202020u;
  return x | ((x & 0x20202020u) * 6u);  // bytes 0..31 stay, 32..63 gain 0xC0
}

// Run j's values as stored for the integer dots: Q5_K and Q6_K unsigned
// (0..31, 0..63; the offsets go through the activation sums), the others
// signed. `P(p)` returns plane p of this row.
template <int TYPE, class Planes>
__device__ inline void plane_run_bytes(const Planes& P, int j, uint32_t (&lo)[4], uint32_t (&hi)[4]) {
  if constexpr (TYPE == kTypeQ8_0) {
    const uint4 a = P(1 + 2 * j), b = P(2 + 2 * j);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      lo[t] = word_of(a, t);
      hi[t] = word_of(b, t);
    }
  } else if constexpr (TYPE == kTypeQ4_0 || TYPE == kTypeIq4Nl) {
    const uint4 a = P(1 + j);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t w = word_of(a, t);
      lo[t] = w & 0x0F0F0F0Fu;
      hi[t] = (w >> 4) & 0x0F0F0F0Fu;
      if constexpr (TYPE == kTypeIq4Nl) {
        lo[t] = iq4_lookup4(lo[t]);
        hi[t] = iq4_lookup4(hi[t]);
      }
    }
  } else if constexpr (TYPE == kTypeQ5K) {
    const int c = j >> 1, sh = 4 * (j & 1);
    const uint4 l0 = P(3 + 2 * c), l1 = P(4 + 2 * c), h0 = P(1), h1 = P(2);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      lo[t] = ((word_of(l0, t) >> sh) & 0x0F0F0F0Fu) | (((word_of(h0, t) >> j) & 0x01010101u) << 4);
      hi[t] = ((word_of(l1, t) >> sh) & 0x0F0F0F0Fu) | (((word_of(h1, t) >> j) & 0x01010101u) << 4);
    }
  } else if constexpr (TYPE == kTypeQ2K) {
    // half h = j / 4 of the 64 quant bytes (planes 1 + 2h, 2 + 2h), field j % 4
    const int h = j >> 2, sh = 2 * (j & 3);
    const uint4 q0 = P(1 + 2 * h), q1 = P(2 + 2 * h);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      lo[t] = (word_of(q0, t) >> sh) & 0x03030303u;
      hi[t] = (word_of(q1, t) >> sh) & 0x03030303u;
    }
  } else if constexpr (TYPE == kTypeQ3K) {
    // 2-bit field j % 4 of half j / 4 (planes 2 + 2h, 3 + 2h), high bit j of
    // the mask (planes 0, 1): values 0..7 standing for value - 4
    const int h = j >> 2, sh = 2 * (j & 3);
    const uint4 q0 = P(2 + 2 * h), q1 = P(3 + 2 * h), m0 = P(0), m1 = P(1);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      lo[t] = ((word_of(q0, t) >> sh) & 0x03030303u) | (((word_of(m0, t) >> j) & 0x01010101u) << 2);
      hi[t] = ((word_of(q1, t) >> sh) & 0x03030303u) | (((word_of(m1, t) >> j) & 0x01010101u) << 2);
    }
  } else {  // Q6_K
    const int h = j >> 2, g = j & 3;
    const int lp = 4 * h + 2 * (g & 1), hp = 8 + 2 * h, ls = 4 * (g >> 1), hs = 2 * g;
    const uint4 l0 = P(lp), l1 = P(lp + 1), h0 = P(hp), h1 = P(hp + 1);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      lo[t] = ((word_of(l0, t) >> ls) & 0x0F0F0F0Fu) | (((word_of(h0, t) >> hs) & 0x03030303u) << 4);
      hi[t] = ((word_of(l1, t) >> ls) & 0x0F0F0F0Fu) | (((word_of(h1, t) >> hs) & 0x03030303u) << 4);
    }
  }
}

// A row's shared-region bytes (Q6_K: d; Q2_K: d | dmin << 16), 0 otherwise.
template <int TYPE>
__device__ inline uint32_t shared_bits(const uint8_t* tile, int r) {
  constexpr int P = plane_count(TYPE), W = plane_shared_width(TYPE);
  if constexpr (W == 2) return *reinterpret_cast<const uint16_t*>(tile + 128 * P + 2 * r);
  if constexpr (W == 4) return *reinterpret_cast<const uint32_t*>(tile + 128 * P + 4 * r);
  return 0u;
}

// Q3_K scale i (0..63, before the -32) from plane 6 (the GGUF packing: low
// nibbles in bytes 0..7, the top two bits in bytes 8..11).
__device__ inline int q3k_scale(const uint4& p6, int i) {
  const uint32_t k1 = 0x03030303u, k2 = 0x0F0F0F0Fu, t = p6.z;
  const int w = i >> 2;
  const uint32_t word = w == 0   ? (p6.x & k2) | ((t & k1) << 4)
                        : w == 1 ? (p6.y & k2) | (((t >> 2) & k1) << 4)
                        : w == 2 ? ((p6.x >> 4) & k2) | (((t >> 4) & k1) << 4)
                                 : ((p6.y >> 4) & k2) | (((t >> 6) & k1) << 4);
  return static_cast<int>(byte_of(word, i & 3));
}

// Signed bytes from 3-bit values 0..7 standing for value - 4 (Q3_K).
__device__ inline uint32_t three_bits_minus_4(uint32_t t) {
  const uint32_t x = t ^ 0x04040404u;
  return x | ((x & 0x04040404u) * 0x3Eu);  // bytes 0..3 stay, 4..7 gain 0xF8
}

// The f16 d of 32-value block j from plane 0 (Q8_0, Q4_0, IQ4_NL).
template <class Planes>
__device__ inline float block_d(const Planes& P, int j) {
  return half_bits(word_of(P(0), j >> 1) >> (16 * (j & 1)));
}

// Q6_K run j's i8 scale of half p.
template <class Planes>
__device__ inline int q6k_scale(const Planes& P, int j, int p) {
  const int i = 8 * (j >> 2) + 2 * (j & 3) + p;
  return static_cast<int8_t>(byte_of(word_of(P(12), i >> 2), i & 3));
}

// Run j as the reference decodes it: signed values and, per half, the f32
// scale and min (scale = d * sub-scale, min = dmin * sub-min).
template <int TYPE, class Planes>
__device__ inline void plane_run_signed(const Planes& P, uint32_t d_bits, int j, uint32_t (&q)[8], float (&scale)[2],
                                        float (&mn)[2]) {
  uint32_t lo[4], hi[4];
  plane_run_bytes<TYPE>(P, j, lo, hi);
  mn[0] = mn[1] = 0.0f;
  if constexpr (TYPE == kTypeQ4_0) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      lo[t] = nibbles_minus_8(lo[t]);
      hi[t] = nibbles_minus_8(hi[t]);
    }
  } else if constexpr (TYPE == kTypeQ6K) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      lo[t] = six_bits_minus_32(lo[t]);
      hi[t] = six_bits_minus_32(hi[t]);
    }
  } else if constexpr (TYPE == kTypeQ3K) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      lo[t] = three_bits_minus_4(lo[t]);
      hi[t] = three_bits_minus_4(hi[t]);
    }
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    q[t] = lo[t];
    q[4 + t] = hi[t];
  }
  if constexpr (TYPE == kTypeQ5K) {
    const uint4 hdr = P(0);
    uint32_t sc, m;
    q4k_sc_m(q4k_six_bit(hdr), j, sc, m);
    scale[0] = scale[1] = half_bits(hdr.x) * static_cast<float>(sc);
    mn[0] = mn[1] = half_bits(hdr.x >> 16) * static_cast<float>(m);
  } else if constexpr (TYPE == kTypeQ6K) {
    const float d = half_bits(d_bits);
    scale[0] = d * static_cast<float>(q6k_scale(P, j, 0));
    scale[1] = d * static_cast<float>(q6k_scale(P, j, 1));
  } else if constexpr (TYPE == kTypeQ2K) {
    const float d = half_bits(d_bits), dmin = half_bits(d_bits >> 16);
    const uint4 sc = P(0);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int i = 8 * (j >> 2) + 2 * (j & 3) + p;
      const uint32_t b = byte_of(word_of(sc, i >> 2), i & 3);
      scale[p] = d * static_cast<float>(b & 0xFu);
      mn[p] = dmin * static_cast<float>(b >> 4);
    }
  } else if constexpr (TYPE == kTypeQ3K) {
    const uint4 p6 = P(6);
    const float d = half_bits(p6.w);
#pragma unroll
    for (int p = 0; p < 2; ++p) scale[p] = d * static_cast<float>(q3k_scale(p6, 8 * (j >> 2) + 2 * (j & 3) + p) - 32);
  } else {
    scale[0] = scale[1] = block_d(P, j);
  }
}

// Repack: thread per (row, group, plane); plane index plane_count(TYPE) is
// the row's shared-region bytes (Q6_K's d at block byte 208, Q2_K's d and
// dmin at 80). Bytes past the block (Q3_K's last plane) and blocks past the
// row's K stay zero.
template <int TYPE>
__global__ void repack_planes_kernel(const uint8_t* __restrict__ raw, uint64_t rows, uint64_t K, uint64_t nb,
                                     uint8_t* __restrict__ tiled) {
  constexpr int P = plane_count(TYPE), BE = block_values(TYPE), BB = block_bytes_of(TYPE);
  constexpr int W = plane_shared_width(TYPE), PT = P + (W ? 1 : 0);
  const uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  if (t >= rows * nb * PT) return;
  const int p = static_cast<int>(t % PT);
  const uint64_t rb = t / PT, b = rb % nb, n = rb / nb;
  const uint64_t blocks = K / BE, row_bytes = blocks * BB;
  const uint8_t* row = raw + n * row_bytes;
  uint8_t* tile = tiled + ((n >> 3) * nb + b) * tile_bytes(TYPE);
  if (p == P) {
    constexpr int src = TYPE == kTypeQ6K ? 208 : 80;
    for (int i = 0; i < W; ++i) tile[128 * P + W * (n & 7) + i] = row[b * BB + src + i];
    return;
  }
  uint8_t* dst = tile + 128 * p + 16 * (n & 7);
  for (int i = 0; i < 16; ++i) {
    uint64_t blk = b, off = 16 * p + i;
    if (BE == 32) {
      if (p == 0) {
        blk = 8 * b + i / 2;
        off = i % 2;
      } else if (TYPE == kTypeQ8_0) {
        blk = 8 * b + (p - 1) / 2;
        off = 2 + 16 * ((p - 1) % 2) + i;
      } else {
        blk = 8 * b + (p - 1);
        off = 2 + i;
      }
    }
    dst[i] = blk < blocks && off < static_cast<uint64_t>(BB) ? row[blk * BB + off] : 0;
  }
}

// Thread per (row, run): value = scale * q - min, product and difference
// each rounded once (quant.rs:1702-1711).
template <int TYPE>
__global__ void dequantize_planes_kernel(const uint8_t* __restrict__ tiled, uint64_t rows, uint64_t K, uint64_t nb,
                                         int logical, float* __restrict__ out) {
  const uint64_t runs = K / 32;
  const uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  if (t >= rows * runs) return;
  const uint64_t u = t % runs, n = t / runs, b = u / 8;
  const int j = static_cast<int>(u % 8), r = static_cast<int>(n & 7);
  const uint8_t* tile = tiled + ((n >> 3) * nb + b) * tile_bytes(TYPE);
  auto planes = [&](int p) { return ld16(tile + 128 * p + 16 * r); };
  const uint32_t d_bits = shared_bits<TYPE>(tile, r);
  uint32_t q[8];
  float scale[2], mn[2];
  plane_run_signed<TYPE>(planes, d_bits, j, q, scale, mn);
  float v[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const float p = scale[i >> 4] * static_cast<float>(static_cast<int8_t>(byte_of(q[i >> 2], i & 3)));
    v[i] = p - mn[i >> 4];
  }
  store_run(out, rows, K, n, 32 * u, logical, v);
}

template <int TYPE>
struct PlaneBlock {
  uint4 p[plane_count(TYPE)];
  uint32_t d_bits;  // Q6_K: this row's f16 d
};

template <int TYPE>
__device__ inline void load_planes(PlaneBlock<TYPE>& a, __amdgpu_buffer_rsrc_t rsrc, uint32_t offset, int r) {
  constexpr int P = plane_count(TYPE);
  const bool none = offset == kBufferNone;
#pragma unroll
  for (int p = 0; p < P; ++p) a.p[p] = buffer_ld16(rsrc, none ? kBufferNone : offset + 128 * p + 16 * r);
  a.d_bits = 0;
  if constexpr (plane_shared_width(TYPE) == 2) {
    const uint32_t w = buffer_ld4(rsrc, none ? kBufferNone : offset + 128 * P + 4 * (r >> 1));
    a.d_bits = (r & 1) ? (w >> 16) : (w & 0xFFFFu);
  } else if constexpr (plane_shared_width(TYPE) == 4) {
    a.d_bits = buffer_ld4(rsrc, none ? kBufferNone : offset + 128 * P + 4 * r);
  }
}

// One run of the int8 GEMV: integer half dots, the format's integer scale
// and offset terms exact, then d_act (and the block's d per run for the
// 32-value formats) in f32.
template <int TYPE, int M>
__device__ inline void plane_run_int8(const PlaneBlock<TYPE>& a, int j, const uint8_t* lds, int kn, int kruns, int bl,
                                      float (&accb)[M], float (&minb)[M]) {
  auto planes = [&](int p) { return a.p[p]; };
  uint32_t lo[4], hi[4];
  plane_run_bytes<TYPE>(planes, j, lo, hi);
  float dj = 0.0f;
  int sc0 = 0, sc1 = 0, smin = 0, smin1 = 0;
  if constexpr (TYPE == kTypeQ5K) {
    uint32_t sc, m;
    q4k_sc_m(q4k_six_bit(a.p[0]), j, sc, m);
    sc0 = static_cast<int>(sc);
    smin = static_cast<int>(m);
  } else if constexpr (TYPE == kTypeQ6K) {
    sc0 = q6k_scale(planes, j, 0);
    sc1 = q6k_scale(planes, j, 1);
  } else if constexpr (TYPE == kTypeQ2K) {
    const int i = 8 * (j >> 2) + 2 * (j & 3);
    const uint32_t b0 = byte_of(word_of(a.p[0], i >> 2), i & 3), b1 = byte_of(word_of(a.p[0], (i + 1) >> 2), (i + 1) & 3);
    sc0 = static_cast<int>(b0 & 0xFu);
    sc1 = static_cast<int>(b1 & 0xFu);
    smin = static_cast<int>(b0 >> 4);
    smin1 = static_cast<int>(b1 >> 4);
  } else if constexpr (TYPE == kTypeQ3K) {
    const int i = 8 * (j >> 2) + 2 * (j & 3);
    sc0 = q3k_scale(a.p[6], i) - 32;
    sc1 = q3k_scale(a.p[6], i + 1) - 32;
  } else {
    dj = block_d(planes, j);
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const uint4* xa = reinterpret_cast<const uint4*>(opaque(lds, m * kn + bl * 256 + 32 * j));
    const uint4 x0 = xa[0], x1 = xa[1];
    int d0 = sdot4(lo[0], x0.x, 0);
    d0 = sdot4(lo[1], x0.y, d0);
    d0 = sdot4(lo[2], x0.z, d0);
    d0 = sdot4(lo[3], x0.w, d0);
    int d1 = sdot4(hi[0], x1.x, 0);
    d1 = sdot4(hi[1], x1.y, d1);
    d1 = sdot4(hi[2], x1.z, d1);
    d1 = sdot4(hi[3], x1.w, d1);
    const uint4 rec = *reinterpret_cast<const uint4*>(opaque(lds, M * kn + 16 * (m * kruns + bl * 8 + j)));
    const float dx = __uint_as_float(rec.x);
    const int s0 = static_cast<int>(rec.y), s1 = static_cast<int>(rec.z);
    if constexpr (TYPE == kTypeQ5K) {
      accb[m] = fmaf(static_cast<float>(sc0 * (d0 + d1)), dx, accb[m]);
      minb[m] = fmaf(static_cast<float>(smin * (s0 + s1)), dx, minb[m]);
    } else if constexpr (TYPE == kTypeQ2K) {
      accb[m] = fmaf(static_cast<float>(sc0 * d0 + sc1 * d1), dx, accb[m]);
      minb[m] = fmaf(static_cast<float>(smin * s0 + smin1 * s1), dx, minb[m]);
    } else if constexpr (TYPE == kTypeQ3K) {
      accb[m] = fmaf(static_cast<float>(sc0 * (d0 - 4 * s0) + sc1 * (d1 - 4 * s1)), dx, accb[m]);
    } else if constexpr (TYPE == kTypeQ6K) {
      accb[m] = fmaf(static_cast<float>(sc0 * (d0 - 32 * s0) + sc1 * (d1 - 32 * s1)), dx, accb[m]);
    } else if constexpr (TYPE == kTypeQ4_0) {
      accb[m] = fmaf(dj * dx, static_cast<float>(d0 + d1 - 8 * (s0 + s1)), accb[m]);
    } else {
      accb[m] = fmaf(dj * dx, static_cast<float>(d0 + d1), accb[m]);
    }
  }
}

template <int TYPE, int M>
__device__ inline void plane_block_int8(const PlaneBlock<TYPE>& a, const uint8_t* lds, int kn, int kruns, int bl,
                                        float (&acc)[M], float (&mins)[M]) {
  float accb[M], minb[M];
#pragma unroll
  for (int m = 0; m < M; ++m) accb[m] = minb[m] = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) plane_run_int8<TYPE, M>(a, j, lds, kn, kruns, bl, accb, minb);
  if constexpr (TYPE == kTypeQ5K) {
    const float d = half_bits(a.p[0].x), dmin = half_bits(a.p[0].x >> 16);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      acc[m] = fmaf(d, accb[m], acc[m]);
      mins[m] = fmaf(dmin, minb[m], mins[m]);
    }
  } else if constexpr (TYPE == kTypeQ2K) {
    const float d = half_bits(a.d_bits), dmin = half_bits(a.d_bits >> 16);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      acc[m] = fmaf(d, accb[m], acc[m]);
      mins[m] = fmaf(dmin, minb[m], mins[m]);
    }
  } else if constexpr (TYPE == kTypeQ6K || TYPE == kTypeQ3K) {
    const float d = half_bits(TYPE == kTypeQ6K ? a.d_bits : a.p[6].w);
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = fmaf(d, accb[m], acc[m]);
  } else {
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] += accb[m];
  }
}

// Decode GEMV over plane tiles, int8 activations staged in LDS (fused
// quantization or pre-quantized), row per lane; the same grid, K-split,
// load order and epilogue as gemv_lds_int8_kernel. K is the logical row
// length (the last group may be partly padding).
template <int TYPE, int M, bool FUSED>
__global__ __launch_bounds__(512) void gemv_planes_int8_kernel(
    const uint8_t* __restrict__ w, int nb, uint64_t rows, uint64_t K, const int8_t* __restrict__ xv,
    const float* __restrict__ xs, const int32_t* __restrict__ xsum, const float* __restrict__ xf,
    float* __restrict__ y, const float* __restrict__ addend, uint64_t addend_stride, SplitK sk) {
  constexpr int kTile = tile_bytes(TYPE);
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = blockDim.x >> 6;
  const int b0 = static_cast<int>(blockIdx.y * nb / sk.ks), b1 = static_cast<int>((blockIdx.y + 1) * nb / sk.ks);
  const int r = lane & 7;
  const uint64_t k0 = static_cast<uint64_t>(b0) * 256;
  const int kn = (b1 - b0) * 256, kruns = kn / 32;
  const int kv = K - k0 < static_cast<uint64_t>(kn) ? static_cast<int>(K - k0) : kn;
  const uint64_t groups = (rows + 7) / 8, group_bytes = static_cast<uint64_t>(nb) * kTile;
  const uint64_t g0 = static_cast<uint64_t>(blockIdx.x) * 8;
  const uint64_t span = (groups - g0 < 8 ? groups - g0 : 8) * group_bytes;
  const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(w + g0 * group_bytes, static_cast<uint32_t>(span));
  const uint32_t lane_off = static_cast<uint32_t>((lane >> 3) * group_bytes);
  auto block_off = [&](int b) { return b < b1 ? lane_off + static_cast<uint32_t>(b) * kTile : kBufferNone; };

  float acc[M], mins[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = mins[m] = 0.0f;
  const int bA = b0 + s;
  bool done = false;
  if constexpr (FUSED && M == 1) {
    // Wave-local staging, as in the Q4_K form (WaveStage; one row here: with
    // two rows the two plane blocks in flight spill): when the rows are
    // whole groups and every wave has at most two blocks (both bounds are
    // work-group uniform), each wave quantizes its own blocks' activations
    // into their LDS slots, with both weight blocks in flight from the
    // start and no work-group barrier before the math.
    if (b1 - b0 <= 2 * S && static_cast<uint64_t>(nb) * 256 == K) {
      const int bB = bA + S;
      WaveStage<TYPE, M, true> ws;
      ws.load(xf, xv, xs, xsum, K, bA, bB, b1, lane);
      PlaneBlock<TYPE> A0, A1;
      load_planes<TYPE>(A0, rsrc, block_off(bA), r);
      load_planes<TYPE>(A1, rsrc, block_off(bB), r);
      ws.put(lds, kn, kruns, b0, bA, bB, b1, lane);
      if (bA < b1) plane_block_int8<TYPE, M>(A0, lds, kn, kruns, bA - b0, acc, mins);
      if (bB < b1) plane_block_int8<TYPE, M>(A1, lds, kn, kruns, bB - b0, acc, mins);
      done = true;
    }
  }
  if (!done) {
    FusedStage<TYPE, M> fs;
    QuantizedStage<TYPE, M> qs;
    if (FUSED)
      fs.load(xf, K, k0, kn, kv);
    else
      qs.load(xv, xs, xsum, K, k0, kn, kv);
    PlaneBlock<TYPE> A;
    load_planes<TYPE>(A, rsrc, block_off(bA), r);
    if (FUSED)
      fs.store(xf, K, k0, kn, kv, lds);
    else
      qs.store(xv, xs, xsum, K, k0, kn, kv, lds);
    __syncthreads();
    for (int b = bA; b < b1; b += S) {
      const PlaneBlock<TYPE> cur = A;
      load_planes<TYPE>(A, rsrc, block_off(b + S), r);
      __builtin_amdgcn_sched_barrier(0);
      plane_block_int8<TYPE, M>(cur, lds, kn, kruns, b - b0, acc, mins);
    }
  }
  finish_rows<M>(acc, mins, rows, y, addend, addend_stride, reinterpret_cast<float*>(lds), sk.partials,
                 sk.counters, sk.ks);
}

// Decode GEMV over plane tiles with f32 activations (the reference's f32
// column loop, quant.rs:559-597: w = scale * q - min, acc += w * x), row per
// lane, waves over the groups; the activations are wave-uniform loads.
template <int TYPE, int M>
__global__ __launch_bounds__(512) void gemv_planes_f32_kernel(const uint8_t* __restrict__ w, int nb, uint64_t rows,
                                                              uint64_t K, const float* __restrict__ x,
                                                              float* __restrict__ y, const float* __restrict__ addend,
                                                              uint64_t addend_stride) {
  constexpr int kTile = tile_bytes(TYPE);
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = blockDim.x >> 6;
  const int r = lane & 7;
  const uint64_t groups = (rows + 7) / 8, group_bytes = static_cast<uint64_t>(nb) * kTile;
  const uint64_t g0 = static_cast<uint64_t>(blockIdx.x) * 8;
  const uint64_t span = (groups - g0 < 8 ? groups - g0 : 8) * group_bytes;
  const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(w + g0 * group_bytes, static_cast<uint32_t>(span));
  const uint32_t lane_off = static_cast<uint32_t>((lane >> 3) * group_bytes);
  float acc[M], mins[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = mins[m] = 0.0f;
  for (int b = s; b < nb; b += S) {
    PlaneBlock<TYPE> a;
    load_planes<TYPE>(a, rsrc, lane_off + static_cast<uint32_t>(b) * kTile, r);
    auto planes = [&](int p) { return a.p[p]; };
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint64_t k = static_cast<uint64_t>(b) * 256 + 32 * j;
      if (k >= K) break;
      uint32_t q[8];
      float scale[2], mn[2];
      plane_run_signed<TYPE>(planes, a.d_bits, j, q, scale, mn);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float4* xr = reinterpret_cast<const float4*>(x + m * K + k);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const float4 xv = xr[t];
          const float xe[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float wv = scale[t >> 2] * static_cast<float>(static_cast<int8_t>(byte_of(q[t], e)));
            wv = wv - mn[t >> 2];
            acc[m] = fmaf(wv, xe[e], acc[m]);
          }
        }
      }
    }
  }
  finish_rows<M>(acc, mins, rows, y, addend, addend_stride, reinterpret_cast<float*>(lds), nullptr, nullptr, 1);
}

// ---------------------------------------------------------------------------
// IQ2 / IQ3 grid formats (src/native/quant.rs:207-277). A weight keeps the
// checkpoint's blocks, stored row after stored row; every format's block is
// an even number of bytes, so blocks are read with 16-bit loads. The grid
// tables are one device-global copy per device, filled by the host
// (mq_set_iq_grids) before any such weight is uploaded.
// ---------------------------------------------------------------------------

__device__ __attribute__((aligned(16))) uint8_t g_iq_grids[kGridTableBytes];

// The format's table within the device copy: byte offset and size.
__host__ __device__ constexpr int grid_table_offset(int type) {
  return type == kTypeIq2Xxs ? kGridIq2Xxs
         : type == kTypeIq2Xs ? kGridIq2Xs
         : type == kTypeIq2S  ? kGridIq2S
         : type == kTypeIq3Xxs ? kGridIq3Xxs
                               : kGridIq3S;
}
__host__ __device__ constexpr int grid_table_size(int type) {
  return type == kTypeIq2Xxs ? 2048 : type == kTypeIq2Xs ? 4096 : type == kTypeIq2S ? 8192 : type == kTypeIq3Xxs ? 1024 : 2048;
}


__device__ inline uint32_t ld_u16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }
__device__ inline uint32_t ld_u32_a2(const uint8_t* p) { return ld_u16(p) | (ld_u16(p + 2) << 16); }

// `iq_signs`: the 7-bit index with its parity in bit 7 (an even number of
// the 8 values is negated).
__device__ inline uint32_t iq_sign_byte(uint32_t index) {
  const uint32_t v = index & 0x7Fu;
  return v | ((static_cast<uint32_t>(__builtin_popcount(v)) & 1u) << 7);
}

// One run of a grid format as `decode` produces it: 32 magnitudes (the grid
// entries' bytes, 4 per word, read as i8), 32 sign bits (bit i negates value
// i: `signed_grid`, quant.rs:60-69) and the two 16-value scales.
struct GridRun {
  uint32_t mag[8];
  uint32_t signs;
  float scale[2];
};

// A run's raw block fields, loaded apart from the decode so that several
// runs' loads can be in flight before any of them is decoded: w = the
// format's words (below), d = the block's f16 d.
struct GridRaw {
  uint32_t w[4];
  uint32_t d;
};

template <int TYPE>
__device__ inline void grid_raw(const uint8_t* __restrict__ blk, int run, GridRaw& r) {
  r.d = ld_u16(blk);
  if constexpr (TYPE == kTypeIq2Xxs) {
    r.w[0] = ld_u32_a2(blk + 2 + 8 * run);  // 4 grid indices
    r.w[1] = ld_u32_a2(blk + 6 + 8 * run);  // 4 x 7 sign bits, 4-bit scale
  } else if constexpr (TYPE == kTypeIq2Xs) {
    r.w[0] = ld_u32_a2(blk + 2 + 8 * run);  // codes 0, 1 (9-bit index, 7 sign bits)
    r.w[1] = ld_u32_a2(blk + 6 + 8 * run);  // codes 2, 3
    r.w[2] = ld_u16(blk + 66 + (run & ~1));  // scale bytes of runs (run & ~1), (run | 1)
  } else if constexpr (TYPE == kTypeIq2S) {
    r.w[0] = ld_u32_a2(blk + 2 + 4 * run);   // 4 low index bytes
    r.w[1] = ld_u32_a2(blk + 34 + 4 * run);  // 4 sign bytes
    r.w[2] = ld_u16(blk + 66 + (run & ~1)) | (ld_u16(blk + 74 + (run & ~1)) << 16);  // qh, scale bytes
  } else if constexpr (TYPE == kTypeIq3Xxs) {
    r.w[0] = ld_u32_a2(blk + 2 + 8 * run);  // grid indices 0..3
    r.w[1] = ld_u32_a2(blk + 6 + 8 * run);  // grid indices 4..7
    r.w[2] = ld_u32_a2(blk + 66 + 4 * run);  // 4 x 7 sign bits, 4-bit scale
  } else {
    static_assert(TYPE == kTypeIq3S, "grid format");
    r.w[0] = ld_u32_a2(blk + 2 + 8 * run);
    r.w[1] = ld_u32_a2(blk + 6 + 8 * run);
    r.w[2] = ld_u32_a2(blk + 74 + 4 * run);  // 4 sign bytes
    r.w[3] = ld_u16(blk + 66 + (run & ~1)) | (ld_u16(blk + 106 + 2 * (run >> 2)) << 16);  // qh, scale nibbles
  }
}

// `table` = the format's grid table (the device copy, or an LDS copy).
template <int TYPE>
__device__ inline void grid_decode(const GridRaw& r, int run, const uint8_t* table, GridRun& g) {
  const float d = half_bits(r.d);
  g.signs = 0;
  if constexpr (TYPE == kTypeIq2Xxs) {
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint2 e = *reinterpret_cast<const uint2*>(table + 8 * ((r.w[0] >> (8 * l)) & 0xFFu));
      g.mag[2 * l] = e.x;
      g.mag[2 * l + 1] = e.y;
      g.signs |= iq_sign_byte(r.w[1] >> (7 * l)) << (8 * l);
    }
    g.scale[0] = g.scale[1] = d * (0.5f + static_cast<float>(r.w[1] >> 28)) * 0.25f;
  } else if constexpr (TYPE == kTypeIq2Xs) {
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint32_t code = (r.w[l >> 1] >> (16 * (l & 1))) & 0xFFFFu;
      const uint2 e = *reinterpret_cast<const uint2*>(table + 8 * (code & 511u));
      g.mag[2 * l] = e.x;
      g.mag[2 * l + 1] = e.y;
      g.signs |= iq_sign_byte(code >> 9) << (8 * l);
    }
    const uint32_t sc = (r.w[2] >> (8 * (run & 1))) & 0xFFu;
    g.scale[0] = d * (0.5f + static_cast<float>(sc & 0xFu)) * 0.25f;
    g.scale[1] = d * (0.5f + static_cast<float>(sc >> 4)) * 0.25f;
  } else if constexpr (TYPE == kTypeIq2S) {
    const uint32_t qh = (r.w[2] >> (8 * (run & 1))) & 0xFFu;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint32_t index = ((r.w[0] >> (8 * l)) & 0xFFu) | (((qh >> (2 * l)) & 3u) << 8);
      const uint2 e = *reinterpret_cast<const uint2*>(table + 8 * index);
      g.mag[2 * l] = e.x;
      g.mag[2 * l + 1] = e.y;
    }
    g.signs = r.w[1];
    const uint32_t sc = (r.w[2] >> (16 + 8 * (run & 1))) & 0xFFu;
    g.scale[0] = d * (0.5f + static_cast<float>(sc & 0xFu)) * 0.25f;
    g.scale[1] = d * (0.5f + static_cast<float>(sc >> 4)) * 0.25f;
  } else if constexpr (TYPE == kTypeIq3Xxs) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      g.mag[i] = *reinterpret_cast<const uint32_t*>(table + 4 * ((r.w[i >> 2] >> (8 * (i & 3))) & 0xFFu));
#pragma unroll
    for (int l = 0; l < 4; ++l) g.signs |= iq_sign_byte(r.w[2] >> (7 * l)) << (8 * l);
    g.scale[0] = g.scale[1] = d * (0.5f + static_cast<float>(r.w[2] >> 28)) * 0.5f;
  } else {
    const uint32_t qh = (r.w[3] >> (8 * (run & 1))) & 0xFFu;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t index = ((r.w[i >> 2] >> (8 * (i & 3))) & 0xFFu) | (((qh >> i) & 1u) << 8);
      g.mag[i] = *reinterpret_cast<const uint32_t*>(table + 4 * index);
    }
    g.signs = r.w[2];
    const uint32_t sc = (r.w[3] >> (16 + 8 * ((run >> 1) & 1) + 4 * (run & 1))) & 0xFu;
    g.scale[0] = g.scale[1] = d * static_cast<float>(1 + 2 * sc);
  }
}

// One run of a grid format as `decode` produces it (src/native/quant.rs:207-277).
template <int TYPE>
__device__ inline void grid_run(const uint8_t* __restrict__ blk, int run, GridRun& g) {
  GridRaw r;
  grid_raw<TYPE>(blk, run, r);
  grid_decode<TYPE>(r, run, g_iq_grids + grid_table_offset(TYPE), g);
}

// Value i of a decoded run: the magnitude as i8, negated (as i8) where its
// sign bit is set.
__device__ inline int grid_value(const GridRun& g, int i) {
  const int8_t m = static_cast<int8_t>(byte_of(g.mag[i >> 2], i & 3));
  return ((g.signs >> i) & 1u) ? static_cast<int8_t>(-m) : m;
}

// Bytes 0xFF where bit b of the 4-bit `s4` is set (byte b), else 0.
__device__ inline uint32_t sign_mask4(uint32_t s4) { return (((s4 & 0xFu) * 0x00204081u) & 0x01010101u) * 0xFFu; }

// Integer dots of a run with 32 int8 activations, per 16-value half:
// sum(+-m a) = sum(m a) - 2 sum over the negated values of m a (exact in
// int32; equal to the reference's i8 values for every magnitude but -128,
// which no grid holds).
__device__ inline void grid_dots(const GridRun& g, const uint32_t (&a)[8], int (&dot)[2]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    int all = 0, neg = 0;
#pragma unroll
    for (int w = 4 * h; w < 4 * h + 4; ++w) {
      all = sdot4(g.mag[w], a[w], all);
      neg = sdot4(g.mag[w] & sign_mask4(g.signs >> (4 * w)), a[w], neg);
    }
    dot[h] = all - 2 * neg;
  }
}

// As grid_dots, with the byte masks of each 8-value group's sign byte read
// from a 256-entry table (`smask8[s]`: byte b of .x / .y is 0xFF where bit
// b / b + 4 of s is set) instead of computed per 4 values. The integer sums
// are the same.
__device__ inline void grid_dots_table(const GridRun& g, const uint32_t (&a)[8], const uint2* smask8,
                                       int (&dot)[2]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    int all = 0, neg = 0;
#pragma unroll
    for (int l = 2 * h; l < 2 * h + 2; ++l) {
      const uint2 mk = smask8[(g.signs >> (8 * l)) & 0xFFu];
      all = sdot4(g.mag[2 * l], a[2 * l], all);
      neg = sdot4(g.mag[2 * l] & mk.x, a[2 * l], neg);
      all = sdot4(g.mag[2 * l + 1], a[2 * l + 1], all);
      neg = sdot4(g.mag[2 * l + 1] & mk.y, a[2 * l + 1], neg);
    }
    dot[h] = all - 2 * neg;
  }
}

template <int TYPE>
__global__ void dequantize_grid_kernel(const uint8_t* __restrict__ w, uint64_t rows, uint64_t nb, int logical,
                                       float* __restrict__ out) {
  constexpr int BB = block_bytes_of(TYPE);
  const uint64_t runs = nb * 8, K = nb * 256;
  const uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  if (t >= rows * runs) return;
  const uint64_t row = t / runs, u = t % runs;
  GridRun g;
  grid_run<TYPE>(w + (row * nb + (u >> 3)) * BB, static_cast<int>(u & 7), g);
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const float v = g.scale[i >> 4] * static_cast<float>(grid_value(g, i));
    const uint64_t col = 32 * u + i;
    if (logical)
      out[col * rows + row] = v;
    else
      out[row * K + col] = v;
  }
}

// Decode GEMV of a grid format (m <= 8): one wave per stored row at a time
// (8 waves per work-group, rows strided over the grid), lanes over the
// row's runs, a fixed-order shuffle reduction. The format's grid table is
// copied to LDS once per work-group, so the four gathers per run leave the
// vector-memory path to the activation and block loads. INT8: the
// reference's int8 path (per half: scale * integer dot, times d_act per
// run); else its f32 column loop (w = scale * q, acc += w * x per value).
// STAGE (int8 mode, when they fit): the int8 activations and their run
// scales are copied to LDS too (m K + 4 m K / 32 bytes), so each row's pass
// reads them from LDS instead of re-reading them through vector memory.
constexpr int kGridGemvWaves = 8;
constexpr int kGridSignTableBytes = 256 * 8;  // sign byte -> byte masks
template <int TYPE, int M, bool INT8, bool STAGE>
__global__ __launch_bounds__(64 * kGridGemvWaves) void gemv_grid_kernel(
    const uint8_t* __restrict__ w, uint64_t nb, uint64_t rows, const int8_t* __restrict__ xv,
    const float* __restrict__ xs, const float* __restrict__ xf, float* __restrict__ y,
    const float* __restrict__ addend, uint64_t addend_stride) {
  static_assert(INT8 || !STAGE, "staging is for the int8 activations");
  constexpr int BB = block_bytes_of(TYPE);
  constexpr int GBYTES = grid_table_size(TYPE);
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  uint8_t* glds = lds;
  // the sign-mask table pays where the grid lookups leave LDS time to spare
  // (measured: IQ2_XS 14.4 -> 12.4 us, IQ2_XXS 12.0 -> 11.5; IQ2_S and IQ3_S,
  // with the most lookups per run, slower by 0.6 / 1.2 us)
  constexpr bool kSignTable = TYPE != kTypeIq2S && TYPE != kTypeIq3S;
  uint2* smask8 = reinterpret_cast<uint2*>(lds + GBYTES);  // kGridSignTableBytes
  const uint64_t runs = nb * 8, K = nb * 256;
  for (int i = threadIdx.x; i < GBYTES / 16; i += 64 * kGridGemvWaves)
    reinterpret_cast<uint4*>(glds)[i] = reinterpret_cast<const uint4*>(g_iq_grids + grid_table_offset(TYPE))[i];
  if (kSignTable && threadIdx.x < 256)
    smask8[threadIdx.x] = make_uint2(sign_mask4(threadIdx.x), sign_mask4(threadIdx.x >> 4));
  const int8_t* xsrc = xv;
  const float* ssrc = xs;
  if constexpr (STAGE) {
    int8_t* xl = reinterpret_cast<int8_t*>(lds + GBYTES + kGridSignTableBytes);
    float* sl = reinterpret_cast<float*>(lds + GBYTES + kGridSignTableBytes + M * K);
    for (uint64_t i = threadIdx.x; i < M * K / 16; i += 64 * kGridGemvWaves)
      reinterpret_cast<uint4*>(xl)[i] = reinterpret_cast<const uint4*>(xv)[i];
    for (uint64_t i = threadIdx.x; i < M * runs / 4; i += 64 * kGridGemvWaves)
      reinterpret_cast<uint4*>(sl)[i] = reinterpret_cast<const uint4*>(xs)[i];
    xsrc = xl;
    ssrc = sl;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  for (uint64_t row = static_cast<uint64_t>(blockIdx.x) * kGridGemvWaves + (threadIdx.x >> 6); row < rows;
       row += static_cast<uint64_t>(gridDim.x) * kGridGemvWaves) {
  const uint8_t* base = w + row * nb * BB;
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.0f;
  // Two runs per lane per pass (u0 and u0 + 64, the order of the one-run
  // loop): both runs' block fields and int8 activations are requested
  // before either is decoded. A second run past the row's end re-reads the
  // first and adds nothing.
  for (uint64_t u0 = lane; u0 < runs; u0 += 128) {
    const bool two = u0 + 64 < runs;
    const uint64_t us[2] = {u0, two ? u0 + 64 : u0};
    GridRaw raw[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) grid_raw<TYPE>(base + (us[q] >> 3) * BB, static_cast<int>(us[q] & 7), raw[q]);
    if constexpr (INT8) {
      uint4 av[2][M][2];
      float as[2][M];
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const uint4* ap = reinterpret_cast<const uint4*>(xsrc + m * K + 32 * us[q]);
          av[q][m][0] = ap[0];
          av[q][m][1] = ap[1];
          as[q][m] = ssrc[m * runs + us[q]];
        }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        GridRun g;
        grid_decode<TYPE>(raw[q], static_cast<int>(us[q] & 7), glds, g);
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const uint32_t a[8] = {av[q][m][0].x, av[q][m][0].y, av[q][m][0].z, av[q][m][0].w,
                                 av[q][m][1].x, av[q][m][1].y, av[q][m][1].z, av[q][m][1].w};
          int dot[2];
          if constexpr (kSignTable)
            grid_dots_table(g, a, smask8, dot);
          else
            grid_dots(g, a, dot);
          float t = g.scale[0] * static_cast<float>(dot[0]);
          t = t + g.scale[1] * static_cast<float>(dot[1]);
          if (q == 0 || two) acc[m] += as[q][m] * t;
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if (q == 1 && !two) break;
        const uint64_t u = us[q];
        GridRun g;
        grid_decode<TYPE>(raw[q], static_cast<int>(u & 7), glds, g);
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const float4* xp = reinterpret_cast<const float4*>(xf + m * K + 32 * u);
#pragma unroll
          for (int q4 = 0; q4 < 8; ++q4) {
            const float4 xq = xp[q4];
            const float xv4[4] = {xq.x, xq.y, xq.z, xq.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int i = 4 * q4 + e;
              const float wv = g.scale[i >> 4] * static_cast<float>(grid_value(g, i));
              acc[m] += wv * xv4[e];
            }
          }
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc[m] += __shfl_xor(acc[m], off);
  if (lane == 0) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float v = acc[m];
      if (addend) v = v + addend[m * addend_stride + row];
      y[m * rows + row] = v;
    }
  }
  }
}

// ---------------------------------------------------------------------------
// Run u of stored row `row` as f32 values, any format: value = scale * q -
// min with the product and difference each rounded once, bit for bit the
// reference's `RunReader::read` + `dequantize_row` arithmetic
// (src/native/quant.rs:308-318, 1702-1711).
// ---------------------------------------------------------------------------
template <int TYPE>
__device__ inline void row_run_values(const uint8_t* __restrict__ tiled, uint64_t nb, uint64_t row, uint64_t u,
                                      float (&v)[32]) {
  const uint64_t b = u >> 3;
  const int j = static_cast<int>(u & 7), r = static_cast<int>(row & 7);
  if constexpr (is_grid_format(TYPE)) {
    GridRun g;
    grid_run<TYPE>(tiled + (row * nb + b) * block_bytes_of(TYPE), j, g);
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = g.scale[i >> 4] * static_cast<float>(grid_value(g, i));
  } else if constexpr (TYPE == kTypeQ4K) {
    const uint8_t* tile = tiled + ((row >> 3) * nb + b) * tile_bytes(TYPE);
    const uint8_t* t = tile + 16 * r;
    const uint4 hdr = ld16(t);
    const int c = j >> 1, shift = 4 * (j & 1);
    const uint4 q0 = ld16(t + 128 * (1 + 2 * c)), q1 = ld16(t + 128 * (2 + 2 * c));
    uint32_t sc, m;
    q4k_sc_m(q4k_six_bit(hdr), j, sc, m);
    const float scale = half_bits(hdr.x) * static_cast<float>(sc);
    const float mn = half_bits(hdr.x >> 16) * static_cast<float>(m);
    const uint32_t words[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float p = scale * static_cast<float>((byte_of(words[i >> 2], i & 3) >> shift) & 0xFu);
      v[i] = p - mn;
    }
  } else if constexpr (TYPE == kTypeIq4Xs) {
    const uint8_t* tile = tiled + ((row >> 3) * nb + b) * tile_bytes(TYPE);
    const uint2 hdr = ld8(tile + 8 * r);
    const uint4 qq = ld16(tile + 64 + 128 * j + 16 * r);
    const float scale = half_bits(hdr.x) * static_cast<float>(iq4xs_ls(hdr, j));
    const uint32_t words[4] = {qq.x, qq.y, qq.z, qq.w};
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4) {
      const uint32_t lo = iq4_lookup4(words[t4] & 0x0F0F0F0Fu), hi = iq4_lookup4((words[t4] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[4 * t4 + e] = scale * static_cast<float>(static_cast<int8_t>(byte_of(lo, e)));
        v[16 + 4 * t4 + e] = scale * static_cast<float>(static_cast<int8_t>(byte_of(hi, e)));
      }
    }
  } else {
    const uint8_t* tile = tiled + ((row >> 3) * nb + b) * tile_bytes(TYPE);
    auto planes = [&](int p) { return ld16(tile + 128 * p + 16 * r); };
    const uint32_t d_bits = shared_bits<TYPE>(tile, r);
    uint32_t q[8];
    float scale[2], mn[2];
    plane_run_signed<TYPE>(planes, d_bits, j, q, scale, mn);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float p = scale[i >> 4] * static_cast<float>(static_cast<int8_t>(byte_of(q[i >> 2], i & 3)));
      v[i] = p - mn[i >> 4];
    }
  }
}

// Embedding of an untransposed packed table (src/native/mod.rs:389-417):
// thread per (token, run), the token's stored row decoded run by run, times
// `scale` when `scaled` (the Kernel's `scale` attribute).
template <int TYPE>
__global__ void embed_rows_kernel(const uint8_t* __restrict__ tiled, uint64_t nb, const uint32_t* __restrict__ ids,
                                  uint64_t count, uint64_t dim, float scale, int scaled, float* __restrict__ out) {
  const uint64_t runs = dim / 32;
  const uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  if (t >= count * runs) return;
  const uint64_t tok = t / runs, u = t % runs;
  float v[32];
  row_run_values<TYPE>(tiled, nb, ids[tok], u, v);
  float4* o = reinterpret_cast<float4*>(out + tok * dim + 32 * u);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float4 q = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    if (scaled) q = make_float4(q.x * scale, q.y * scale, q.z * scale, q.w * scale);
    o[i] = q;
  }
}

// Embedding of a transposed table (stored [dim][vocab]): the token's value
// in every stored row (`quant::element`, src/native/quant.rs:1690-1698).
template <int TYPE>
__global__ void embed_columns_kernel(const uint8_t* __restrict__ tiled, uint64_t nb, const uint32_t* __restrict__ ids,
                                     uint64_t count, uint64_t dim, float scale, int scaled, float* __restrict__ out) {
  const uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  if (t >= count * dim) return;
  const uint64_t tok = t / dim, j = t % dim;
  const uint32_t id = ids[tok];
  float v[32];
  row_run_values<TYPE>(tiled, nb, j, id >> 5, v);
  float x = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) x = (static_cast<int>(id & 31) == i) ? v[i] : x;
  out[tok * dim + j] = scaled ? x * scale : x;
}

// Input-major (axpy) product (src/native/quant.rs:1652-1688): the stored
// rows are the K input rows, each holding N output columns. Thread per (run
// of 32 columns, half); work-group column y = a K-split; each row j adds
// x[r][j] * value for every row r whose x[r][j] is not zero (the reference
// skips zero activations), f32 multiply then add. Partials [ks][MM][N].
template <int TYPE, int MM>
__global__ __launch_bounds__(256) void axpy_kernel(const uint8_t* __restrict__ tiled, uint64_t nb, uint64_t K,
                                                   uint64_t N, const float* __restrict__ x, int rows, uint64_t kchunk,
                                                   float* __restrict__ part) {
  const uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  const uint64_t u = t >> 1;
  const int h = static_cast<int>(t & 1);
  if (u >= N / 32) return;
  const uint64_t ks = blockIdx.y, j0 = ks * kchunk, j1 = j0 + kchunk < K ? j0 + kchunk : K;
  float acc[MM][16];
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[m][i] = 0.0f;
  for (uint64_t j = j0; j < j1; ++j) {
    float v[32];
    row_run_values<TYPE>(tiled, nb, j, u, v);
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const float xv = m < rows ? x[m * K + j] : 0.0f;
      if (xv != 0.0f) {
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[m][i] += xv * (h ? v[16 + i] : v[i]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    float4* o = reinterpret_cast<float4*>(part + (ks * MM + m) * N + 32 * u + 16 * h);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = make_float4(acc[m][4 * i], acc[m][4 * i + 1], acc[m][4 * i + 2], acc[m][4 * i + 3]);
  }
}

// y[r][n] = sum over the K-splits in split order [+ addend].
__global__ void axpy_finish_kernel(const float* __restrict__ part, int ks, int mm, int rows, uint64_t N,
                                   float* __restrict__ y, const float* __restrict__ addend, uint64_t addend_stride) {
  const uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  if (t >= static_cast<uint64_t>(rows) * N) return;
  const uint64_t r = t / N, n = t % N;
  float s = part[r * N + n];
  for (int i = 1; i < ks; ++i) s += part[(static_cast<uint64_t>(i) * mm + r) * N + n];
  if (addend) s = s + addend[r * addend_stride + n];
  y[r * N + n] = s;
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
                                                   const float* __restrict__ addend, uint64_t addend_stride,
                                                   uint64_t kdim, F16Range rg) {
  __shared__ __attribute__((aligned(16))) uint16_t As[kBM][kLdsK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[kBN][kLdsK];
  __shared__ float row_fac[kBM];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const uint64_t m0 = static_cast<uint64_t>(blockIdx.y) * kBM;
  if (tid < kBM) row_fac[tid] = out_factor(rg, m0 + tid, m_rows);  // read after the loop's barriers
  const uint64_t n0 = static_cast<uint64_t>(blockIdx.x) * kBN;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const uint64_t K = kdim;  // the logical row length (a multiple of 32)
  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int ksteps = static_cast<int>((K + kBK - 1) / kBK);
  for (int kb = 0; kb < ksteps; ++kb) {
    // A tile: 128 rows x 64 halves, 16 B per chunk, 4 chunks per thread.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int idx = tid + 256 * i;
      int row = idx >> 3, ch = idx & 7;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (m0 + row < m_rows && static_cast<uint64_t>(kb) * kBK + ch * 8 < K)
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
        if constexpr (is_plane_format(TYPE)) {
          // run 2c + h: values 0..15 at k = 32h, 16..31 at 32h + 16
          const uint8_t* tile = w + ((n >> 3) * nb + b) * tile_bytes(TYPE);
          const int r = static_cast<int>(n & 7);
          auto planes = [&](int p) { return ld16(tile + 128 * p + 16 * r); };
          const uint32_t d_bits = shared_bits<TYPE>(tile, r);
          uint32_t q[8];
          float sc[2], mn[2];
          plane_run_signed<TYPE>(planes, d_bits, 2 * c + h, q, sc, mn);
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const float s = sc[t >> 2] * rg.up, m = mn[t >> 2] * rg.up;
            out[2 * t] = pack_f16x2(fmaf(s, static_cast<float>(static_cast<int8_t>(byte_of(q[t], 0))), -m),
                                    fmaf(s, static_cast<float>(static_cast<int8_t>(byte_of(q[t], 1))), -m));
            out[2 * t + 1] = pack_f16x2(fmaf(s, static_cast<float>(static_cast<int8_t>(byte_of(q[t], 2))), -m),
                                        fmaf(s, static_cast<float>(static_cast<int8_t>(byte_of(q[t], 3))), -m));
          }
        } else if constexpr (TYPE == kTypeQ4K) {
          const uint8_t* tile = w + ((n >> 3) * nb + b) * kQ4kTileBytes + (n & 7) * 16;
          const uint4 hdr = ld16(tile);
          const uint4 qq = ld16(tile + 128 * (1 + 2 * c + h));
          const Q4kSixBit six = q4k_six_bit(hdr);
          uint32_t sc0, mm0, sc1, mm1;
          q4k_sc_m(six, 2 * c, sc0, mm0);
          q4k_sc_m(six, 2 * c + 1, sc1, mm1);
          const float d = half_bits(hdr.x) * rg.up, dmin = half_bits(hdr.x >> 16) * rg.up;
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
          const float sj = half_bits(hdr.x) * rg.up * static_cast<float>(iq4xs_ls(hdr, j));
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
      const int k_hi = TYPE == kTypeQ4K ? 32 + 16 * h : 32 * h + 16;  // IQ4_XS and plane formats alike
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
    float rf[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) rf[e] = row_fac[wm + 16 * i + 4 * (lane >> 4) + e];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint64_t col = n0 + wn + 16 * j + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint64_t row = m0 + wm + 16 * i + 4 * (lane >> 4) + e;
        if (row < m_rows && col < rows) {
          float v = acc[i][j][e] * rf[e];
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
// 64-wide K-step (one Q4_K quant chunk = two runs). The weight bytes of the
// next super-block (4 K-steps) are in flight while the current one is
// multiplied, to cover HBM latency.
//
// Operand lanes: lane = i + 16 * kq holds rows/columns i and k = 8 kq .. 8 kq + 7
// of the 32-wide MFMA K, for A and B alike; the weight bytes 8 kq .. 8 kq + 7
// of a chunk give run 2c's k-slot (low nibbles) and run 2c+1's (high).
// ---------------------------------------------------------------------------

// One lane's raw weight bytes for one super-block and NF fragments.
template <int TYPE, int NF>
struct RawB {
  uint4 hdr[NF];
  uint2 qa[4][NF];  // Q4_K: chunk c bytes 8kq..8kq+7; IQ4_XS: run 2c's 8 index bytes
  uint2 qb[4][NF];  // IQ4_XS: run 2c+1's 8 index bytes (unused for Q4_K)
};

template <int TYPE, int NF>
__device__ inline void load_raw_b(RawB<TYPE, NF>& r, const uint8_t* const (&tile0)[NF], const bool (&live)[NF],
                                  uint64_t b, int kq) {
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    if (!live[f]) {
      r.hdr[f] = make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int c = 0; c < 4; ++c) r.qa[c][f] = r.qb[c][f] = make_uint2(0, 0);
      continue;
    }
    const uint8_t* tile = tile0[f] + b * tile_bytes(TYPE);
    if (TYPE == kTypeQ4K) {
      r.hdr[f] = ld16(tile);
#pragma unroll
      for (int c = 0; c < 4; ++c) r.qa[c][f] = ld8(tile + 128 * (1 + 2 * c + (kq >> 1)) + 8 * (kq & 1));
    } else {
      // tile0 points at this row's header; planes start 64 bytes into the
      // tile at 16 bytes per row (the row index is folded into tile0).
      const uint2 h = ld8(tile);
      r.hdr[f] = make_uint4(h.x, h.y, 0, 0);
    }
  }
}

template <int NF>
__device__ inline void load_raw_b_iq4(RawB<kTypeIq4Xs, NF>& r, const uint8_t* const (&planes0)[NF],
                                      const bool (&live)[NF], uint64_t b) {
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    if (!live[f]) continue;
    const uint8_t* pl = planes0[f] + b * kIq4xsTileBytes;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      r.qa[c][f] = ld8(pl + 128 * (2 * c));
      r.qb[c][f] = ld8(pl + 128 * (2 * c + 1));
    }
  }
}

template <int TYPE, int NF, int C>
__device__ inline void dequant_b(const RawB<TYPE, NF>& r, int kq, float up, half8 (&bop)[2][NF]) {
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    uint32_t p0[4], p1[4];
    if (TYPE == kTypeQ4K) {
      const Q4kSixBit six = q4k_six_bit(r.hdr[f]);
      uint32_t sc0, mm0, sc1, mm1;
      q4k_sc_m(six, 2 * C, sc0, mm0);
      q4k_sc_m(six, 2 * C + 1, sc1, mm1);
      const float d = half_bits(r.hdr[f].x) * up, dmin = half_bits(r.hdr[f].x >> 16) * up;
      const float s0 = d * static_cast<float>(sc0), s1 = d * static_cast<float>(sc1);
      const float n0m = -(dmin * static_cast<float>(mm0)), n1m = -(dmin * static_cast<float>(mm1));
      const uint2 qa = r.qa[C][f];
      const uint32_t lo[2] = {qa.x & 0x0F0F0F0Fu, qa.y & 0x0F0F0F0Fu};
      const uint32_t hi[2] = {(qa.x >> 4) & 0x0F0F0F0Fu, (qa.y >> 4) & 0x0F0F0F0Fu};
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
    } else {
      const uint2 h2 = make_uint2(r.hdr[f].x, r.hdr[f].y);
      const float d = half_bits(h2.x) * up;
      const float sa = d * static_cast<float>(iq4xs_ls(h2, 2 * C));
      const float sb = d * static_cast<float>(iq4xs_ls(h2, 2 * C + 1));
      const int sh = 4 * (kq >> 1);  // low nibbles hold weights 0..15, high 16..31
      const uint2 qa = r.qa[C][f], qb = r.qb[C][f];
      const uint32_t ia[2] = {iq4_lookup4((qa.x >> sh) & 0x0F0F0F0Fu), iq4_lookup4((qa.y >> sh) & 0x0F0F0F0Fu)};
      const uint32_t ib[2] = {iq4_lookup4((qb.x >> sh) & 0x0F0F0F0Fu), iq4_lookup4((qb.y >> sh) & 0x0F0F0F0Fu)};
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
    }
    bop[0][f] = *reinterpret_cast<half8*>(p0);
    bop[1][f] = *reinterpret_cast<half8*>(p1);
  }
}

// Plane formats on the register-B GEMM: one lane's bytes of one group (256
// values of its weight row) for the values 8 kq .. 8 kq + 7 of every run
// (its K slot of the 32-wide MFMA K), loaded one group ahead.
//  Q8_0: q[j] = run j's 8 quants; hdr = plane 0 (the 8 d).
//  Q4_0 / IQ4_NL: q[j] = run j's 8 nibble-pair bytes (low nibbles hold
//   values 0..15, high 16..31); hdr = plane 0.
//  Q5_K: q[c] = chunk c's 8 nibble bytes (runs 2c, 2c + 1); hb[0] = the 8
//   high-bit bytes; hdr = d, dmin, scales.
//  Q6_K: q[2h + g % 2] = low-nibble bytes of half h; hb[h] = its high-bit
//   bytes; hdr = the 16 i8 scales; dsh = d.
template <int TYPE, int NF>
struct RawPB {
  uint4 hdr[NF];
  uint2 q[8][NF];
  uint2 hb[2][NF];
  uint32_t dsh[NF];
};

template <int TYPE, int NF>
__device__ inline void load_raw_pb(RawPB<TYPE, NF>& r, const uint8_t* const (&tile0)[NF], const int (&row)[NF],
                                   const bool (&live)[NF], uint64_t b, int kq) {
  constexpr int P = plane_count(TYPE);
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    if (!live[f]) {
      r.hdr[f] = make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 8; ++j) r.q[j][f] = make_uint2(0, 0);
      r.hb[0][f] = r.hb[1][f] = make_uint2(0, 0);
      r.dsh[f] = 0;
      continue;
    }
    const uint8_t* t = tile0[f] + b * tile_bytes(TYPE);
    const int R = row[f], off = 16 * R + 8 * (kq & 1), hp = kq >> 1;
    if constexpr (TYPE == kTypeQ8_0) {
      r.hdr[f] = ld16(t + 16 * R);
#pragma unroll
      for (int j = 0; j < 8; ++j) r.q[j][f] = ld8(t + 128 * (1 + 2 * j + hp) + off);
    } else if constexpr (TYPE == kTypeQ4_0 || TYPE == kTypeIq4Nl) {
      r.hdr[f] = ld16(t + 16 * R);
#pragma unroll
      for (int j = 0; j < 8; ++j) r.q[j][f] = ld8(t + 128 * (1 + j) + off);
    } else if constexpr (TYPE == kTypeQ5K) {
      r.hdr[f] = ld16(t + 16 * R);
#pragma unroll
      for (int c = 0; c < 4; ++c) r.q[c][f] = ld8(t + 128 * (3 + 2 * c + hp) + off);
      r.hb[0][f] = ld8(t + 128 * (1 + hp) + off);
    } else if constexpr (TYPE == kTypeQ2K) {
      r.hdr[f] = ld16(t + 16 * R);
#pragma unroll
      for (int h = 0; h < 2; ++h) r.q[h][f] = ld8(t + 128 * (1 + 2 * h + hp) + off);
      r.dsh[f] = *reinterpret_cast<const uint32_t*>(t + 128 * P + 4 * R);
    } else if constexpr (TYPE == kTypeQ3K) {
      r.hdr[f] = ld16(t + 128 * 6 + 16 * R);
#pragma unroll
      for (int h = 0; h < 2; ++h) r.q[h][f] = ld8(t + 128 * (2 + 2 * h + hp) + off);
      r.hb[0][f] = ld8(t + 128 * hp + off);
    } else {
      r.hdr[f] = ld16(t + 128 * 12 + 16 * R);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        r.q[2 * h][f] = ld8(t + 128 * (4 * h + hp) + off);
        r.q[2 * h + 1][f] = ld8(t + 128 * (4 * h + 2 + hp) + off);
        r.hb[h][f] = ld8(t + 128 * (8 + 2 * h + hp) + off);
      }
      r.dsh[f] = *reinterpret_cast<const uint16_t*>(t + 128 * P + 2 * R);
    }
  }
}

// K-step C (runs 2C, 2C + 1) of the plane formats as MFMA B operands:
// value = scale * q - min, rounded once to f16.
template <int TYPE, int NF, int C>
__device__ inline void dequant_pb(const RawPB<TYPE, NF>& r, int kq, float up, half8 (&bop)[2][NF]) {
#pragma unroll
  for (int f = 0; f < NF; ++f) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = 2 * C + h;
      uint32_t v[2];
      float sc, mn = 0.0f;
      if constexpr (TYPE == kTypeQ8_0) {
        v[0] = r.q[j][f].x;
        v[1] = r.q[j][f].y;
        sc = half_bits(word_of(r.hdr[f], j >> 1) >> (16 * (j & 1)));
      } else if constexpr (TYPE == kTypeQ4_0 || TYPE == kTypeIq4Nl) {
        const int sh = 4 * (kq >> 1);
        const uint32_t n0 = (r.q[j][f].x >> sh) & 0x0F0F0F0Fu, n1 = (r.q[j][f].y >> sh) & 0x0F0F0F0Fu;
        if constexpr (TYPE == kTypeQ4_0) {
          v[0] = nibbles_minus_8(n0);
          v[1] = nibbles_minus_8(n1);
        } else {
          v[0] = iq4_lookup4(n0);
          v[1] = iq4_lookup4(n1);
        }
        sc = half_bits(word_of(r.hdr[f], j >> 1) >> (16 * (j & 1)));
      } else if constexpr (TYPE == kTypeQ5K) {
        const uint2 w = r.q[C][f], hb = r.hb[0][f];
        v[0] = ((w.x >> (4 * h)) & 0x0F0F0F0Fu) | (((hb.x >> j) & 0x01010101u) << 4);
        v[1] = ((w.y >> (4 * h)) & 0x0F0F0F0Fu) | (((hb.y >> j) & 0x01010101u) << 4);
        uint32_t s6, m6;
        q4k_sc_m(q4k_six_bit(r.hdr[f]), j, s6, m6);
        sc = half_bits(r.hdr[f].x) * static_cast<float>(s6);
        mn = half_bits(r.hdr[f].x >> 16) * static_cast<float>(m6);
      } else if constexpr (TYPE == kTypeQ2K) {
        const int hh = j >> 2, sh = 2 * (j & 3);
        v[0] = (r.q[hh][f].x >> sh) & 0x03030303u;
        v[1] = (r.q[hh][f].y >> sh) & 0x03030303u;
        const int si = 8 * hh + 2 * (j & 3) + (kq >> 1);
        const uint32_t b = byte_of(word_of(r.hdr[f], si >> 2), si & 3);
        sc = half_bits(r.dsh[f]) * static_cast<float>(b & 0xFu);
        mn = half_bits(r.dsh[f] >> 16) * static_cast<float>(b >> 4);
      } else if constexpr (TYPE == kTypeQ3K) {
        const int hh = j >> 2, sh = 2 * (j & 3);
        const uint2 hb = r.hb[0][f];
        v[0] = three_bits_minus_4(((r.q[hh][f].x >> sh) & 0x03030303u) | (((hb.x >> j) & 0x01010101u) << 2));
        v[1] = three_bits_minus_4(((r.q[hh][f].y >> sh) & 0x03030303u) | (((hb.y >> j) & 0x01010101u) << 2));
        sc = half_bits(r.hdr[f].w) * static_cast<float>(q3k_scale(r.hdr[f], 8 * hh + 2 * (j & 3) + (kq >> 1)) - 32);
      } else {
        const int hh = j >> 2, g = j & 3;
        const uint2 w = r.q[2 * hh + (g & 1)][f], hb = r.hb[hh][f];
        const int ls = 4 * (g >> 1), hs = 2 * g;
        v[0] = six_bits_minus_32(((w.x >> ls) & 0x0F0F0F0Fu) | (((hb.x >> hs) & 0x03030303u) << 4));
        v[1] = six_bits_minus_32(((w.y >> ls) & 0x0F0F0F0Fu) | (((hb.y >> hs) & 0x03030303u) << 4));
        const int si = 8 * hh + 2 * g + (kq >> 1);
        sc = half_bits(r.dsh[f]) * static_cast<float>(static_cast<int8_t>(byte_of(word_of(r.hdr[f], si >> 2), si & 3)));
      }
      sc *= up;
      mn *= up;
      uint32_t p[4];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        p[2 * t] = pack_f16x2(fmaf(sc, static_cast<float>(static_cast<int8_t>(byte_of(v[t], 0))), -mn),
                              fmaf(sc, static_cast<float>(static_cast<int8_t>(byte_of(v[t], 1))), -mn));
        p[2 * t + 1] = pack_f16x2(fmaf(sc, static_cast<float>(static_cast<int8_t>(byte_of(v[t], 2))), -mn),
                                  fmaf(sc, static_cast<float>(static_cast<int8_t>(byte_of(v[t], 3))), -mn));
      }
      bop[h][f] = *reinterpret_cast<half8*>(p);
    }
  }
}

template <int TYPE, int MF, int NF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NF == 2 ? 2 : 1))) void gemm_rb_kernel(const uint8_t* __restrict__ w, int nb, uint64_t rows,
                                                      uint64_t rows_padded, const uint16_t* __restrict__ a16,
                                                      uint64_t m_rows, float* __restrict__ y,
                                                      const float* __restrict__ addend, uint64_t addend_stride,
                                                      F16Range rg) {
  constexpr int BM = MF * 16;
  constexpr int LDK = kBK + 8;  // halves per LDS row (16-byte pad)
  constexpr int A_CHUNKS = BM * kBK / 8 / 256;  // 16-byte chunks per thread per K-step
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM][LDK];
  __shared__ float row_fac[BM];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int li = lane & 15, kq = lane >> 4;
  const uint64_t m0 = static_cast<uint64_t>(blockIdx.y) * BM;
  const uint64_t n0 = static_cast<uint64_t>(blockIdx.x) * (4 * NF * 16) + static_cast<uint64_t>(wave) * NF * 16;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  const float my_fac = tid < BM ? out_factor(rg, m0 + tid, m_rows) : 0.0f;
  // split-K over gridDim.z work-groups: super-blocks [bl, bh) of the row,
  // results to the split's own [m_rows][rows] slice of y (the partials,
  // which the host sums in split order)
  const int bl = static_cast<int>(blockIdx.z * static_cast<uint64_t>(nb) / gridDim.z);
  const int bh = static_cast<int>((blockIdx.z + 1) * static_cast<uint64_t>(nb) / gridDim.z);
  const int ksteps = bh * 4;  // K-step indices are absolute
  y += static_cast<uint64_t>(blockIdx.z) * m_rows * rows;

  floatx4 acc[MF][NF];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int f = 0; f < NF; ++f) acc[i][f] = floatx4{0.f, 0.f, 0.f, 0.f};

  // this lane's weight row per fragment: header address in super-block 0,
  // and (IQ4_XS) the start of its quant planes; plane formats: the tile
  // and the row within it
  const uint8_t* tile0[NF];
  const uint8_t* planes0[NF];
  int prow[NF];
  bool wlive[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const uint64_t n = n0 + 16 * f + li;
    wlive[f] = n < rows_padded;
    const uint64_t nn = wlive[f] ? n : 0;
    const uint8_t* t = w + (nn >> 3) * nb * tile_bytes(TYPE);
    prow[f] = static_cast<int>(nn & 7);
    tile0[f] = is_plane_format(TYPE) ? t : t + (nn & 7) * (TYPE == kTypeQ4K ? 16 : 8);
    planes0[f] = t + 64 + (nn & 7) * 16 + 8 * (kq & 1);
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

  using Raw = std::conditional_t<is_plane_format(TYPE), RawPB<TYPE, NF>, RawB<TYPE, NF>>;
  auto load_b = [&](Raw& r, uint64_t b) {
    if constexpr (is_plane_format(TYPE)) {
      load_raw_pb<TYPE, NF>(r, tile0, prow, wlive, b, kq);
    } else {
      load_raw_b<TYPE, NF>(r, tile0, wlive, b, kq);
      if constexpr (TYPE == kTypeIq4Xs) load_raw_b_iq4<NF>(r, planes0, wlive, b);
    }
  };
  // Pipeline: the activations of K-step kb + 2 are loaded into registers
  // during K-step kb (areg[kb & 1]) and stored to the other LDS buffer at
  // the end of K-step kb + 1; the next super-block's weights are loaded
  // during the block's second K-step, after that step's activation load.
  // So each wait for a load (vector memory returns in issue order) comes
  // about two K-steps after it was issued, and the barrier between K-steps
  // waits for LDS only, not for the loads in flight.
  Raw cur, nxt;
  uint4 areg[2][A_CHUNKS];
  load_a(4 * bl, areg[0]);
  if (4 * bl + 1 < ksteps) load_a(4 * bl + 1, areg[1]);
  load_b(nxt, static_cast<uint64_t>(bl));
  store_a(0, areg[0]);  // K-step 4 bl is even: buffer 0
  if (tid < BM) row_fac[tid] = my_fac;
  __syncthreads();

  // ld: the registers of K-step kb's parity (free: stored at the end of
  // K-step kb - 1), st: those of kb + 1
  auto kstep = [&](int kb, const half8 (&bop)[2][NF], uint4 (&ld)[A_CHUNKS], uint4 (&st)[A_CHUNKS], int b_next) {
    const int buf = kb & 1;
    if (kb + 2 < ksteps) load_a(kb + 2, ld);
    if (b_next >= 0) load_b(nxt, static_cast<uint64_t>(b_next));
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
    if (kb + 1 < ksteps) store_a(buf ^ 1, st);
    lds_barrier();
  };

  for (int b = bl; b < bh; ++b) {
    cur = nxt;
    const int b_next = b + 1 < bh ? b + 1 : -1;
    half8 bop[2][NF];
    if constexpr (is_plane_format(TYPE)) {
      dequant_pb<TYPE, NF, 0>(cur, kq, rg.up, bop);
      kstep(4 * b + 0, bop, areg[0], areg[1], -1);
      dequant_pb<TYPE, NF, 1>(cur, kq, rg.up, bop);
      kstep(4 * b + 1, bop, areg[1], areg[0], b_next);
      dequant_pb<TYPE, NF, 2>(cur, kq, rg.up, bop);
      kstep(4 * b + 2, bop, areg[0], areg[1], -1);
      dequant_pb<TYPE, NF, 3>(cur, kq, rg.up, bop);
      kstep(4 * b + 3, bop, areg[1], areg[0], -1);
    } else {
      dequant_b<TYPE, NF, 0>(cur, kq, rg.up, bop);
      kstep(4 * b + 0, bop, areg[0], areg[1], -1);
      dequant_b<TYPE, NF, 1>(cur, kq, rg.up, bop);
      kstep(4 * b + 1, bop, areg[1], areg[0], b_next);
      dequant_b<TYPE, NF, 2>(cur, kq, rg.up, bop);
      kstep(4 * b + 2, bop, areg[0], areg[1], -1);
      dequant_b<TYPE, NF, 3>(cur, kq, rg.up, bop);
      kstep(4 * b + 3, bop, areg[1], areg[0], -1);
    }
  }

#pragma unroll
  for (int i = 0; i < MF; ++i) {
    float rf[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) rf[e] = row_fac[16 * i + 4 * kq + e];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint64_t col = n0 + 16 * f + li;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint64_t row = m0 + 16 * i + 4 * kq + e;
        if (row < m_rows && col < rows) {
          float v = acc[i][f][e] * rf[e];
          if (addend) v = v + addend[row * addend_stride + col];
          y[row * rows + col] = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Q4_K prefill GEMM, K-split form (`gemm_ks_kernel`).
//
// 512 threads = 8 waves, two per SIMD: wave = nw + 4 kw. A work-group owns a
// 128 (M) x 256 (N) output tile; wave (nw, kw) computes its 128 x 64 part over
// the K half kw (super-blocks [kw nbh, (kw + 1) nbh)) on v_mfma_f32_32x32x16_f16,
// and the two halves are summed through LDS at the end. Splitting K inside the
// work-group gives 224 work-groups at 512 x 14336 (one per CU) with two waves
// per SIMD, so one wave's dequantization overlaps the other's MFMAs.
//
// A (f16 activations): per K half a 4-stage LDS ring, one 64-wide K-step
//   (128 rows x 128 B) per stage, filled 3 K-steps ahead by buffer_load ... lds
//   (16 B chunks XOR-swizzled by row so the 32 rows of a fragment read hit
//   distinct banks). One barrier per K-step, issued without a vmcnt(0) fence:
//   each wave waits only for the stage it reads next.
// B (Q4_K weight rows): each lane holds column 32 f + l32 of its 64 and the K
//   slot 8 kh .. 8 kh + 7 of every 16-wide MFMA slice; the chunk bytes (two
//   8-byte pieces per fragment) are loaded 3 K-steps ahead, the super-block
//   header one super-block ahead. Operands are dequantized one slice ahead of
//   their MFMAs: value = s q - m is computed as s (1024 + q) + (-m - 1024 s)
//   on the f16 1024 + q that a byte permute builds from the nibble
//   (v_fma_mix, f32 arithmetic, one rounding to f16); high nibbles use
//   s / 16 on 1024 + 16 q.
// ---------------------------------------------------------------------------

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kKsThreads = 512;
constexpr int kKsBM = 128, kKsBN = 256;
constexpr int kKsStage = kKsBM * 128;  // bytes per A stage
constexpr int kKsDma = 4;              // 1 KB buffer_load ... lds per wave per stage

// 16 bytes per lane from a buffer straight into LDS (lane l writes lds + 16 l);
// voffset per lane, soffset uniform.
__device__ inline void lds_dma16_so(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voffset, uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds), 16,
                                           static_cast<int>(voffset), static_cast<int>(soffset), 0, 0);
}

__device__ inline uint2 buffer_ld8_so(__amdgpu_buffer_rsrc_t r, uint32_t voffset, uint32_t soffset) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(voffset), static_cast<int>(soffset), 0);
  return make_uint2(v.x, v.y);
}

__device__ inline uint4 buffer_ld16_so(__amdgpu_buffer_rsrc_t r, uint32_t voffset, uint32_t soffset) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voffset), static_cast<int>(soffset), 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// gfx9 s_waitcnt immediate for vmcnt(n) alone (expcnt 7, lgkmcnt 15 = no wait)
constexpr int wait_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

// Work-group barrier without the memory fence __syncthreads() adds (which
// waits for every outstanding load); the clobber keeps memory operations on
// their side of it.
__device__ inline void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }

// f16 pair (lo, hi) = s * x.lo + c, s * x.hi + c for the f16 halves of x,
// computed in f32 and rounded once.
__device__ inline uint32_t fma_mix_pair(float s, uint32_t x, float c) {
  uint32_t r;
  asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(s), "v"(x), "v"(c));
  asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "+v"(r) : "v"(s), "v"(x), "v"(c));
  return r;
}

struct KsScales {
  float s[2][2], c[2][2];  // [run of the chunk][fragment]
};

// Scales of chunk C (runs 2C, 2C + 1) for both fragments.
template <int C>
__device__ inline void ks_scales(const uint4 (&hdr)[2], float up, KsScales& cs) {
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const Q4kSixBit six = q4k_six_bit(hdr[f]);
    uint32_t sc0, mm0, sc1, mm1;
    q4k_sc_m(six, 2 * C, sc0, mm0);
    q4k_sc_m(six, 2 * C + 1, sc1, mm1);
    const float d = half_bits(hdr[f].x) * up, dmin = half_bits(hdr[f].x >> 16) * up;
    const float s0 = d * static_cast<float>(sc0), s1 = d * static_cast<float>(sc1) * 0.0625f;
    cs.s[0][f] = s0;
    cs.s[1][f] = s1;
    cs.c[0][f] = fmaf(-1024.0f, s0, -(dmin * static_cast<float>(mm0)));
    cs.c[1][f] = fmaf(-1024.0f, s1, -(dmin * static_cast<float>(mm1)));
  }
}

// Slice SL (16 K values) of a chunk: run SL >> 1, chunk bytes 16 (SL & 1) + 8 kh
// .. + 7 (q[f] = the two 8-byte pieces: .xy bytes 8 kh.., .zw bytes 16 + 8 kh..).
template <int SL>
__device__ inline void ks_slice(const uint4 (&q)[2], const KsScales& cs, half8 (&bop)[2]) {
  constexpr int run = SL >> 1;
  const uint32_t mask = run ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const uint32_t x0 = ((SL & 1) ? q[f].z : q[f].x) & mask, x1 = ((SL & 1) ? q[f].w : q[f].y) & mask;
    const float s = cs.s[run][f], c = cs.c[run][f];
    uint32_t p[4];
    // bytes (x.b0, 0x64, x.b1, 0x64) and (x.b2, 0x64, x.b3, 0x64): f16 1024 + byte
    p[0] = fma_mix_pair(s, __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u), c);
    p[1] = fma_mix_pair(s, __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u), c);
    p[2] = fma_mix_pair(s, __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u), c);
    p[3] = fma_mix_pair(s, __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u), c);
    bop[f] = *reinterpret_cast<half8*>(p);
  }
}

__global__ __launch_bounds__(kKsThreads) void gemm_ks_kernel(const uint8_t* __restrict__ w, int nb, uint64_t rows,
                                                              uint64_t rows_padded, const uint16_t* __restrict__ a16,
                                                              uint64_t m_rows, float* __restrict__ y,
                                                              const float* __restrict__ addend,
                                                              uint64_t addend_stride, F16Range rg) {
  constexpr int MF = 4, NF = 2, D = kKsDma;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * 4 * kKsStage];  // [kw][stage]
  __shared__ __attribute__((aligned(16))) float row_fac[kKsBM];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int nw = wave & 3, kw = wave >> 2;
  const int l32 = lane & 31, kh = lane >> 5;
  const uint64_t m0 = static_cast<uint64_t>(blockIdx.y) * kKsBM;
  // the tile's output factors: loaded before the weight and activation
  // prefetches, so the prologue's vmcnt wait covers them
  const float my_fac = tid < kKsBM ? out_factor(rg, m0 + tid, m_rows) : 0.0f;
  const uint64_t n0 = static_cast<uint64_t>(blockIdx.x) * kKsBN + static_cast<uint64_t>(nw) * 64;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  // split-K over gridDim.z: super-blocks [zb0, zb1) of the row, the
  // partials to the split's own [m_rows][rows] slice of y (summed in split
  // order afterwards); the two K halves divide that range
  const int zb0 = static_cast<int>(blockIdx.z * static_cast<uint64_t>(nb) / gridDim.z);
  const int zb1 = static_cast<int>((blockIdx.z + 1) * static_cast<uint64_t>(nb) / gridDim.z);
  const int nbh = (zb1 - zb0 + 1) / 2, sb0 = zb0 + kw * nbh;
  const int sb_end = sb0 + nbh < zb1 ? sb0 + nbh : zb1;  // this half's super-blocks [sb0, sb_end)
  const int ksteps = 4 * nbh;                            // K-steps per half (both halves run as many)
  y += static_cast<uint64_t>(blockIdx.z) * m_rows * rows;
  uint8_t* const ring = lds + kw * 4 * kKsStage;
  auto swz = [](int row) { return (row >> 1) & 7; };

  // A: the tile's rows as one buffer resource (rows past m_rows read zeros)
  const uint64_t a_rows = m_rows - m0 < static_cast<uint64_t>(kKsBM) ? m_rows - m0 : kKsBM;
  const __amdgpu_buffer_rsrc_t rsA = buffer_rsrc(a16 + m0 * K, static_cast<uint32_t>(a_rows * K * 2));
  uint32_t a_off[D];  // this lane's 16 bytes of each of its DMA instructions: row, swizzled chunk
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int row = 8 * (nw * D + d) + (lane >> 3), cs = lane & 7;
    a_off[d] = static_cast<uint32_t>(row * K * 2 + (cs ^ swz(row)) * 16);
  }
  uint32_t a_rd[4][MF];  // fragment i, slice sl: row 32 i + l32, chunk 2 sl + kh
#pragma unroll
  for (int sl = 0; sl < 4; ++sl)
#pragma unroll
    for (int i = 0; i < MF; ++i) {
      const int row = 32 * i + l32, c = 2 * sl + kh;
      a_rd[sl][i] = row * 128 + ((c ^ swz(row)) * 16);
    }

  // B: this wave's 64 weight rows = 8 row groups
  const uint64_t groups = rows_padded / 8, group_bytes = static_cast<uint64_t>(nb) * kQ4kTileBytes;
  const uint64_t wg0 = n0 / 8;
  const uint64_t wspan = wg0 < groups ? (groups - wg0 < 4 * NF ? groups - wg0 : 4 * NF) * group_bytes : 0;
  const __amdgpu_buffer_rsrc_t rsB =
      buffer_rsrc(w + (wg0 < groups ? wg0 : 0) * group_bytes, static_cast<uint32_t>(wspan));
  uint32_t b_lane[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int nl = 32 * f + l32;
    b_lane[f] = static_cast<uint32_t>((nl >> 3) * group_bytes) + (nl & 7) * 16;
  }
  // local K-step j = chunk j % 4 of super-block sb0 + j / 4
  // Per-lane offsets stay in VGPRs; the K position goes in the uniform
  // soffset, and steps past this half's super-blocks read through a
  // zero-length resource (zeros), so the loads cost no per-lane selects.
  const __amdgpu_buffer_rsrc_t rsZ = buffer_rsrc(w, 0);
  uint32_t b_q[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) b_q[f] = b_lane[f] + 128 + 8 * kh;
  auto load_chunk = [&](uint4 (&q)[NF], int j) {
    const int sb = sb0 + j / 4, c = j % 4;
    const __amdgpu_buffer_rsrc_t rs = j < ksteps && sb < sb_end ? rsB : rsZ;
    const uint32_t so = static_cast<uint32_t>(sb) * kQ4kTileBytes + 256 * c;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint2 lo = buffer_ld8_so(rs, b_q[f], so);
      const uint2 hi = buffer_ld8_so(rs, b_q[f] + 128, so);
      q[f] = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
  };
  auto load_hdr = [&](uint4 (&h)[NF], int bl) {
    const int sb = sb0 + bl;
    const __amdgpu_buffer_rsrc_t rs = bl < nbh && sb < sb_end ? rsB : rsZ;
#pragma unroll
    for (int f = 0; f < NF; ++f) h[f] = buffer_ld16_so(rs, b_lane[f], static_cast<uint32_t>(sb) * kQ4kTileBytes);
  };
  const __amdgpu_buffer_rsrc_t rsAZ = buffer_rsrc(a16, 0);
  auto dma = [&](int stage, int j) {
    const __amdgpu_buffer_rsrc_t rs = j < ksteps && sb0 + j / 4 < sb_end ? rsA : rsAZ;
    const uint32_t so = static_cast<uint32_t>(4 * sb0 + j) * 128;
#pragma unroll
    for (int d = 0; d < D; ++d) lds_dma16_so(rs, ring + stage * kKsStage + (nw * D + d) * 1024, a_off[d], so);
  };
  auto read_a = [&](int stage, int sl, half8 (&dst)[MF]) {
#pragma unroll
    for (int i = 0; i < MF; ++i) dst[i] = *reinterpret_cast<const half8*>(ring + stage * kKsStage + a_rd[sl][i]);
  };

  floatx16 acc[MF][NF];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][f][e] = 0.f;

  uint4 hb[2][NF];  // headers of the even / odd local super-blocks
  uint4 qb[4][NF];  // chunk bytes, buffer j % 4
  // issue order (vmcnt): header, chunks 0..2, stages 0..2
  load_hdr(hb[0], 0);
  load_chunk(qb[0], 0);
  load_chunk(qb[1], 1);
  load_chunk(qb[2], 2);
  dma(0, 0);
  dma(1, 1);
  dma(2, 2);
  __builtin_amdgcn_s_waitcnt(wait_vmcnt(2 * D));  // stage 0 (and every B load) complete
  if (tid < kKsBM) row_fac[tid] = my_fac;  // read in the epilogue, after the K loop's barriers
  wg_barrier();
  half8 af[MF], an[MF], bc[NF], bn[NF];
  read_a(0, 0, af);
  KsScales sc_cur, sc_nxt;
  ks_scales<0>(hb[0], rg.up, sc_cur);
  ks_slice<0>(qb[0], sc_cur, bc);

  // Slice SL of K-step j = 4 bl + C: read the next slice's A, dequantize the
  // next slice's B, 8 MFMAs on the current ones. (Raising the wave priority
  // around the MFMAs measured slower, 72-78 against 69 us at
  // 512 x 14336 x 4096, and so did one barrier per two K-steps with the ring
  // filled two stages at a time, 72-78 us: its extra live registers spill.)
#define MQ_KS_SLICE(C, HB, SL)                                                                 \
  {                                                                                            \
    if (SL < 3) read_a(C, SL + 1, an); else read_a((C + 1) % 4, 0, an);                        \
    if (SL < 3) {                                                                              \
      ks_slice<(SL + 1) % 4>(qb[C], sc_cur, bn);                                               \
    } else {                                                                                   \
      if (C < 3) ks_scales<(C + 1) % 4>(hb[HB], rg.up, sc_nxt); else ks_scales<0>(hb[HB ^ 1], rg.up, sc_nxt); \
      ks_slice<0>(qb[(C + 1) % 4], sc_nxt, bn);                                                \
    }                                                                                          \
    _Pragma("unroll") for (int i = 0; i < MF; ++i)                                             \
      _Pragma("unroll") for (int f = 0; f < NF; ++f)                                           \
        acc[i][f] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bc[f], acc[i][f], 0, 0, 0);  \
    _Pragma("unroll") for (int i = 0; i < MF; ++i) af[i] = an[i];                              \
    _Pragma("unroll") for (int f = 0; f < NF; ++f) bc[f] = bn[f];                              \
  }
  // K-step j = 4 bl + C: chunk bytes in qb[C], header of super-block bl in hb[HB].
  // Issue order per K-step: chunk j + 3 (4 loads), at C == 1 header bl + 1 (2),
  // then after two slices the wait for stage j + 1, the barrier and stage j + 3
  // (4 DMAs). At that wait the newest 8 loads are this K-step's B loads and
  // (part of) stage j + 2, so vmcnt(8) completes stage j + 1 for this wave; the
  // barrier makes it complete for all waves of the half.
#define MQ_KS_STEP(C, HB)                                                                      \
  {                                                                                            \
    const int j = 4 * bl + C;                                                                  \
    load_chunk(qb[(C + 3) % 4], j + 3);                                                        \
    if (C == 1) load_hdr(hb[HB ^ 1], bl + 1);                                                  \
    MQ_KS_SLICE(C, HB, 0)                                                                      \
    MQ_KS_SLICE(C, HB, 1)                                                                      \
    __builtin_amdgcn_s_waitcnt(wait_vmcnt(2 * D));                                             \
    wg_barrier();                                                                              \
    dma((C + 3) % 4, j + 3);                                                                   \
    MQ_KS_SLICE(C, HB, 2)                                                                      \
    MQ_KS_SLICE(C, HB, 3)                                                                      \
    sc_cur = sc_nxt;                                                                           \
  }
  // One super-block per iteration: the next block's header arrives in hb[1]
  // during the block (used from its last slice on) and moves to hb[0] at its
  // end. Bodies of two and four blocks (fewer loop heads, where the compiler
  // waits for every load in flight) measured slower at 512 x 14336 x 4096
  // (78.0 and 80.5 us against 72.3 us), and a half of one block no longer
  // runs a block of zeros.
  for (int bl = 0; bl < nbh; ++bl) {
    MQ_KS_STEP(0, 0)
    MQ_KS_STEP(1, 0)
    MQ_KS_STEP(2, 0)
    MQ_KS_STEP(3, 0)
#pragma unroll
    for (int f = 0; f < NF; ++f) hb[0][f] = hb[1][f];
  }
#undef MQ_KS_STEP
#undef MQ_KS_SLICE

  // The K halves meet in LDS, and the tile leaves through it: wave (nw, 1)
  // hands its accumulators to wave (nw, 0) (16-byte LDS writes and reads in
  // fragment order), which adds them, applies the row factors and writes the
  // 128 x 64 part row-major into the ring; then all eight waves store whole
  // rows, 16 bytes per lane (a 1 KB row per wave store). Stores of 4 bytes per
  // lane from half the waves held the epilogue at about 7 us per tile. Every
  // wave's DMAs (including the zero-filled ones past the end) must land
  // before the ring is reused.
  __builtin_amdgcn_s_waitcnt(wait_vmcnt(0));
  wg_barrier();
  float4* const red = reinterpret_cast<float4*>(lds + nw * 32768);
  float* const tile = reinterpret_cast<float*>(lds);  // [kKsBM][kKsBN]
  if (kw == 1) {
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          red[((i * NF + f) * 4 + g) * 64 + lane] =
              make_float4(acc[i][f][4 * g], acc[i][f][4 * g + 1], acc[i][f][4 * g + 2], acc[i][f][4 * g + 3]);
  }
  lds_barrier();
  if (kw == 0) {
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 o = red[((i * NF + f) * 4 + g) * 64 + lane];
          acc[i][f][4 * g] += o.x;
          acc[i][f][4 * g + 1] += o.y;
          acc[i][f][4 * g + 2] += o.z;
          acc[i][f][4 * g + 3] += o.w;
        }
  }
  lds_barrier();
  // D layout (32 x 32): lane holds column l32, rows 8 g + 4 kh + e of fragment element 4 g + e
  if (kw == 0) {
    const int tc = 64 * nw + l32;
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 rf4 = *reinterpret_cast<const float4*>(&row_fac[32 * i + 8 * g + 4 * kh]);
        const float rf[4] = {rf4.x, rf4.y, rf4.z, rf4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 32 * i + 8 * g + 4 * kh + e;
#pragma unroll
          for (int f = 0; f < NF; ++f) tile[r * kKsBN + tc + 32 * f] = acc[i][f][4 * g + e] * rf[e];
        }
      }
  }
  lds_barrier();
  const uint64_t c0 = static_cast<uint64_t>(blockIdx.x) * kKsBN + 4 * lane;  // this lane's first column
  if (rows % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0 && addend == nullptr &&
      (blockIdx.x + 1) * static_cast<uint64_t>(kKsBN) <= rows) {
    // every column of the tile in range, 16-byte aligned rows, no addend; the
    // final output (not split partials, which the sum kernel reads next) is
    // stored nontemporally (about 1-1.5 us less per launch)
    typedef float f32x4 __attribute__((ext_vector_type(4)));
#pragma unroll 4
    for (int it = 0; it < kKsBM / 8; ++it) {
      const int r = 8 * it + wave;
      if (m0 + r >= m_rows) break;  // uniform
      const float4 v = *reinterpret_cast<const float4*>(&tile[r * kKsBN + 4 * lane]);
      float* const dst = y + (m0 + r) * rows + c0;
      if (gridDim.z == 1)
        __builtin_nontemporal_store(f32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4*>(dst));
      else
        *reinterpret_cast<float4*>(dst) = v;
    }
  } else {
    for (int it = 0; it < kKsBM / 8; ++it) {
      const int r = 8 * it + wave;
      const uint64_t row = m0 + r;
      if (row >= m_rows) break;  // uniform
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (c0 + c < rows) {
          float o = tile[r * kKsBN + 4 * lane + c];
          if (addend) o = o + addend[row * addend_stride + c0 + c];
          y[row * rows + c0 + c] = o;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Grid-format prefill GEMM, `gemm_grid_kernel<F, MF, NF>` (IQ2_XXS, IQ2_XS,
// IQ2_S, IQ3_XXS, IQ3_S; src/native/quant.rs:207-277 decode).
//
// The register-B structure of gemm_rb_kernel: a 16 MF x 64 NF output tile
// per work-group (4 waves side by side in N), A (f16 activations)
// double-buffered through LDS, B decoded per lane. Lane (li, kq) of a
// v_mfma_f32_16x16x32_f16 holds column li and K values 8 kq .. 8 kq + 7 of a
// 32-value run: exactly grid group kq of that run (one 8-magnitude IQ2
// entry, or two 4-magnitude IQ3 entries), its sign byte and the scale of
// half kq >> 1. So each lane reads only its group's block fields (16-bit
// loads of the raw blocks, one super-block ahead). The format's grid table
// and a sign-byte -> f16 sign-mask table are copied to LDS at start.
//
// B = +-(scale * magnitude) rounded once to f16: the magnitude byte becomes
// the f16 1024 + m by a byte permute, v_fma_mix forms s (1024 + m) - 1024 s
// = s m in f32 (exact before its one rounding, 1024 s being exact) and
// rounds it to f16, and the sign is an xor of the f16 sign bit. This reads
// the magnitudes as unsigned bytes; the host routes a weight here only when
// every byte of its grid table is below 128, where that equals the i8
// reading of `grid_value`.
// ---------------------------------------------------------------------------

// Raw block fields of one lane's group for DEPTH K-steps (2 DEPTH runs),
// per fragment: a = index bytes, b = sign / aux word, c = per-run-pair
// bytes (qh, scales; at the pair's even slot). K-step C of a super-block
// sits in ring slot C % DEPTH. The block's f16 d is kept apart.
template <int NF, int DEPTH>
struct RawG {
  uint32_t a[NF][2 * DEPTH], b[NF][2 * DEPTH], c[NF][2 * DEPTH];
};

// Ring depth in K-steps: half a super-block for the formats with three
// fields per run (registers) and for IQ2_XXS (measured: M = 512 GEMM 181 ->
// 166 us), a whole one for the others.
__host__ __device__ constexpr int grid_ring_depth(int type) {
  return type == kTypeIq2S || type == kTypeIq3S || type == kTypeIq2Xxs ? 2 : 4;
}

template <int TYPE, int NF>
__device__ inline void load_d_g(uint32_t (&d)[NF], const uint8_t* const (&blk0)[NF], uint64_t b) {
#pragma unroll
  for (int f = 0; f < NF; ++f) d[f] = ld_u16(blk0[f] + b * block_bytes_of(TYPE));
}

// Runs 2C and 2C + 1 of super-block b (K-step C of the block), into ring
// slot C % DEPTH.
template <int TYPE, int NF, int DEPTH, int C>
__device__ inline void load_raw_g(RawG<NF, DEPTH>& r, const uint8_t* const (&blk0)[NF], uint64_t b, int l) {
  constexpr int BB = block_bytes_of(TYPE);
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const uint8_t* p = blk0[f] + b * BB;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = 2 * C + h, q = 2 * (C % DEPTH) + h;
      if constexpr (TYPE == kTypeIq2Xxs) {
        r.a[f][q] = ld_u16(p + 2 + 8 * j + 2 * (l >> 1));
        r.b[f][q] = ld_u32_a2(p + 6 + 8 * j);
      } else if constexpr (TYPE == kTypeIq2Xs) {
        r.a[f][q] = ld_u16(p + 2 + 2 * (4 * j + l));
        if ((j & 1) == 0) r.c[f][q] = ld_u16(p + 66 + j);
      } else if constexpr (TYPE == kTypeIq2S) {
        r.a[f][q] = ld_u16(p + 2 + 4 * j + 2 * (l >> 1));
        r.b[f][q] = ld_u16(p + 34 + 4 * j + 2 * (l >> 1));
        if ((j & 1) == 0) r.c[f][q] = ld_u16(p + 66 + j) | (ld_u16(p + 74 + j) << 16);
      } else if constexpr (TYPE == kTypeIq3Xxs) {
        r.a[f][q] = ld_u16(p + 2 + 8 * j + 2 * l);
        r.b[f][q] = ld_u32_a2(p + 66 + 4 * j);
      } else {
        static_assert(TYPE == kTypeIq3S, "grid format");
        r.a[f][q] = ld_u16(p + 2 + 8 * j + 2 * l);
        r.b[f][q] = ld_u16(p + 74 + 4 * j + 2 * (l >> 1));
        if ((j & 1) == 0) r.c[f][q] = ld_u16(p + 66 + j) | (ld_u16(p + 106 + 2 * (j >> 2)) << 16);
      }
    }
  }
}

// Run j, group l of every fragment as an f16 B operand (the same fields
// and scale arithmetic as grid_run).
template <int TYPE, int NF, int DEPTH>
__device__ inline void dequant_g(const RawG<NF, DEPTH>& r, const uint32_t (&dbits)[NF], int j, int q, int l,
                                 const uint8_t* glds, const uint4* smask, float up, half8 (&bop)[NF]) {
  const uint2* g64 = reinterpret_cast<const uint2*>(glds);
  const uint32_t* g32 = reinterpret_cast<const uint32_t*>(glds);
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const float d = half_bits(dbits[f]) * up;
    uint32_t m0, m1, sg;
    float s;
    if constexpr (TYPE == kTypeIq2Xxs) {
      const uint32_t aux = r.b[f][q];
      const uint2 e = g64[(r.a[f][q] >> (8 * (l & 1))) & 0xFFu];
      m0 = e.x;
      m1 = e.y;
      sg = iq_sign_byte(aux >> (7 * l));
      s = d * (0.5f + static_cast<float>(aux >> 28)) * 0.25f;
    } else if constexpr (TYPE == kTypeIq2Xs) {
      const uint32_t code = r.a[f][q];
      const uint2 e = g64[code & 511u];
      m0 = e.x;
      m1 = e.y;
      sg = iq_sign_byte(code >> 9);
      const uint32_t sc = (r.c[f][q & ~1] >> (8 * (j & 1))) & 0xFFu;
      s = d * (0.5f + static_cast<float>((sc >> (4 * (l >> 1))) & 0xFu)) * 0.25f;
    } else if constexpr (TYPE == kTypeIq2S) {
      const uint32_t cc = r.c[f][q & ~1];
      const uint32_t qh = (cc >> (8 * (j & 1))) & 0xFFu;
      const uint2 e = g64[((r.a[f][q] >> (8 * (l & 1))) & 0xFFu) | (((qh >> (2 * l)) & 3u) << 8)];
      m0 = e.x;
      m1 = e.y;
      sg = (r.b[f][q] >> (8 * (l & 1))) & 0xFFu;
      const uint32_t sc = (cc >> (16 + 8 * (j & 1))) & 0xFFu;
      s = d * (0.5f + static_cast<float>((sc >> (4 * (l >> 1))) & 0xFu)) * 0.25f;
    } else if constexpr (TYPE == kTypeIq3Xxs) {
      const uint32_t a = r.a[f][q], aux = r.b[f][q];
      m0 = g32[a & 0xFFu];
      m1 = g32[(a >> 8) & 0xFFu];
      sg = iq_sign_byte(aux >> (7 * l));
      s = d * (0.5f + static_cast<float>(aux >> 28)) * 0.5f;
    } else {
      const uint32_t a = r.a[f][q], cc = r.c[f][q & ~1];
      const uint32_t qh = (cc >> (8 * (j & 1))) & 0xFFu;
      m0 = g32[(a & 0xFFu) | (((qh >> (2 * l)) & 1u) << 8)];
      m1 = g32[((a >> 8) & 0xFFu) | (((qh >> (2 * l + 1)) & 1u) << 8)];
      sg = (r.b[f][q] >> (8 * (l & 1))) & 0xFFu;
      const uint32_t sc = (cc >> (16 + 8 * ((j >> 1) & 1) + 4 * (j & 1))) & 0xFu;
      s = d * static_cast<float>(1 + 2 * sc);
    }
    const float c = -1024.0f * s;
    const uint4 sm = smask[sg];
    uint32_t p[4];
    p[0] = fma_mix_pair(s, __builtin_amdgcn_perm(0x64646464u, m0, 0x04010400u), c) ^ sm.x;
    p[1] = fma_mix_pair(s, __builtin_amdgcn_perm(0x64646464u, m0, 0x04030402u), c) ^ sm.y;
    p[2] = fma_mix_pair(s, __builtin_amdgcn_perm(0x64646464u, m1, 0x04010400u), c) ^ sm.z;
    p[3] = fma_mix_pair(s, __builtin_amdgcn_perm(0x64646464u, m1, 0x04030402u), c) ^ sm.w;
    bop[f] = *reinterpret_cast<half8*>(p);
  }
}

// (128 x 128 tiles: held to two waves per SIMD, so that one work-group's
// decode overlaps the other's MFMAs)
template <int TYPE, int MF, int NF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NF == 2 ? 2 : 1))) void gemm_grid_kernel(const uint8_t* __restrict__ w, int nb, uint64_t rows,
                                                        const uint16_t* __restrict__ a16, uint64_t m_rows,
                                                        float* __restrict__ y, const float* __restrict__ addend,
                                                        uint64_t addend_stride, F16Range rg) {
  constexpr int BM = MF * 16;
  constexpr int LDK = kBK + 8;                  // halves per LDS row (16-byte pad)
  constexpr int A_CHUNKS = BM * kBK / 8 / 256;  // 16-byte chunks per thread per K-step
  constexpr int GBYTES = grid_table_size(TYPE);
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM][LDK];
  __shared__ __attribute__((aligned(16))) uint8_t glds[GBYTES];
  __shared__ uint4 smask[256];
  __shared__ float row_fac[BM];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int li = lane & 15, kq = lane >> 4;
  const uint64_t m0 = static_cast<uint64_t>(blockIdx.y) * BM;
  const float my_fac = tid < BM ? out_factor(rg, m0 + tid, m_rows) : 0.0f;
  const uint64_t n0 = static_cast<uint64_t>(blockIdx.x) * (4 * NF * 16) + static_cast<uint64_t>(wave) * NF * 16;
  const uint64_t K = static_cast<uint64_t>(nb) * 256;
  // split-K over gridDim.z: super-blocks [bl, bh), results to the split's
  // own [m_rows][rows] slice of y (partials summed by the host)
  const int bl = static_cast<int>(blockIdx.z * static_cast<uint64_t>(nb) / gridDim.z);
  const int bh = static_cast<int>((blockIdx.z + 1) * static_cast<uint64_t>(nb) / gridDim.z);
  const int ksteps = bh * 4;  // K-step indices are absolute
  y += static_cast<uint64_t>(blockIdx.z) * m_rows * rows;

  floatx4 acc[MF][NF];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int f = 0; f < NF; ++f) acc[i][f] = floatx4{0.f, 0.f, 0.f, 0.f};

  // this lane's stored row per fragment (columns past the last row read the
  // last row; their outputs are not stored)
  const uint8_t* blk0[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const uint64_t n = n0 + 16 * f + li;
    blk0[f] = w + (n < rows ? n : rows - 1) * static_cast<uint64_t>(nb) * block_bytes_of(TYPE);
  }

  // the format's grid table, and per sign byte the xor masks of its four
  // f16 pairs (bit 2p -> bit 15 of word p, bit 2p + 1 -> bit 31)
  for (int i = tid; i < GBYTES / 16; i += 256)
    reinterpret_cast<uint4*>(glds)[i] = reinterpret_cast<const uint4*>(g_iq_grids + grid_table_offset(TYPE))[i];
  {
    uint32_t v[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) v[p] = (((tid >> (2 * p)) & 1u) << 15) | (((tid >> (2 * p + 1)) & 1u) << 31);
    smask[tid] = make_uint4(v[0], v[1], v[2], v[3]);
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

  // raw fields: K-step slot C of the block in use is refilled with the next
  // block's as soon as it is decoded (a super-block ahead, one copy)
  constexpr int DEPTH = grid_ring_depth(TYPE);
  RawG<NF, DEPTH> raw;
  uint32_t dcur[NF], dnxt[NF];
  const uint64_t b0 = static_cast<uint64_t>(bl);
  load_d_g<TYPE, NF>(dcur, blk0, b0);
  load_raw_g<TYPE, NF, DEPTH, 0>(raw, blk0, b0, kq);
  load_raw_g<TYPE, NF, DEPTH, 1>(raw, blk0, b0, kq);
  if constexpr (DEPTH == 4) {
    load_raw_g<TYPE, NF, DEPTH, 2>(raw, blk0, b0, kq);
    load_raw_g<TYPE, NF, DEPTH, 3>(raw, blk0, b0, kq);
  }
  uint4 areg[A_CHUNKS];
  load_a(4 * bl, areg);
  store_a(0, areg);  // K-step 4 bl is even: buffer 0
  if (tid < BM) row_fac[tid] = my_fac;
  __syncthreads();

  auto kstep = [&](int kb, const half8 (&bop)[2][NF]) {
    const int buf = kb & 1;
    const bool more = kb + 1 < ksteps;
    if (more) load_a(kb + 1, areg);
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
  };

  auto step = [&](int b, auto cc) {
    constexpr int C = decltype(cc)::value, Q = 2 * (C % DEPTH);
    half8 bop[2][NF];
    dequant_g<TYPE, NF, DEPTH>(raw, dcur, 2 * C, Q, kq, glds, smask, rg.up, bop[0]);
    dequant_g<TYPE, NF, DEPTH>(raw, dcur, 2 * C + 1, Q + 1, kq, glds, smask, rg.up, bop[1]);
    // refill the slot with K-step C + DEPTH (this block's, or the next's)
    constexpr int CN = (C + DEPTH) % 4;
    const int bn = b + (C + DEPTH) / 4;
    if (bn < bh) load_raw_g<TYPE, NF, DEPTH, CN>(raw, blk0, static_cast<uint64_t>(bn), kq);
    kstep(4 * b + C, bop);
  };
  for (int b = bl; b < bh; ++b) {
    const bool more = b + 1 < bh;
    if (more) load_d_g<TYPE, NF>(dnxt, blk0, static_cast<uint64_t>(b + 1));
    step(b, std::integral_constant<int, 0>{});
    step(b, std::integral_constant<int, 1>{});
    step(b, std::integral_constant<int, 2>{});
    step(b, std::integral_constant<int, 3>{});
    if (more) {
#pragma unroll
      for (int f = 0; f < NF; ++f) dcur[f] = dnxt[f];
    }
  }

#pragma unroll
  for (int i = 0; i < MF; ++i) {
    float rf[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) rf[e] = row_fac[16 * i + 4 * kq + e];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint64_t col = n0 + 16 * f + li;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint64_t row = m0 + 16 * i + 4 * kq + e;
        if (row < m_rows && col < rows) {
          float v = acc[i][f][e] * rf[e];
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
                                 int32_t* sums, hipStream_t stream) {
  uint64_t total = m * k;
  hipLaunchKernelGGL(quantize_act_kernel, dim3(grid_for(total / 4, 256)), dim3(256), 0, stream, x, total,
                     values, scales, sums);
}

void launch_activations_f16(const float* x, uint64_t m, uint64_t k, int int8, uint16_t* a16, float* row_factor,
                            hipStream_t stream) {
  const uint64_t held = (k / 4 + 255) / 256;
  switch (held) {
#define X(H)                                                                                                     \
  case H:                                                                                                        \
    hipLaunchKernelGGL(activations_f16_kernel<H>, dim3(static_cast<unsigned>(m)), dim3(256), 0, stream, x, k, int8, \
                       a16, row_factor);                                                                         \
    return;
    X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(9) X(10) X(11) X(12) X(13) X(14) X(15) X(16)
#undef X
    default:
      hipLaunchKernelGGL(activations_f16_kernel<0>, dim3(static_cast<unsigned>(m)), dim3(256), 0, stream, x, k, int8,
                         a16, row_factor);
  }
}

void weight_f16_factors(float amax, float* up, float* down) {
  int e = 0;
  if (amax > 0.0f && std::isfinite(amax)) {
    int ex = 0;
    (void)std::frexp(amax, &ex);
    e = 15 - ex;  // the weight's exponent range lies within [-40, 40]
    e = e < -40 ? -40 : (e > 40 ? 40 : e);
  }
  *up = std::ldexp(1.0f, e);
  *down = std::ldexp(1.0f, -e);
}

void launch_absmax(const float* x, uint64_t n, uint32_t* out, hipStream_t stream) {
  uint64_t groups = grid_for(n / 4, 256);
  if (groups > 1024) groups = 1024;
  if (groups == 0) return;
  hipLaunchKernelGGL(absmax_kernel, dim3(static_cast<unsigned>(groups)), dim3(256), 0, stream, x, n, out);
}

int gemv_default_splits(uint64_t rows, uint64_t nb, uint64_t m, int variant) {
  if (variant == 0) variant = 3;
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

namespace {

// Bytes of dynamic LDS the LDS-staged GEMV needs for a K range of nbk
// super-blocks: the activations (int8 values + per-run f32) or the
// cross-wave reduction, whichever is larger.
size_t gemv_lds_bytes(int type, uint64_t nbk, uint64_t m, int splits) {
  const size_t act = type == kTypeQ4K ? m * nbk * 256 + m * nbk * 8 * 8 : m * nbk * 256 + m * nbk * 8 * 4;
  const size_t red = static_cast<size_t>(splits) * m * 2 * 64 * 4;
  return act > red ? act : red;
}

int lds_form_max_splits(uint64_t) { return 8; }  // launch bound 512

// The 16-row form, when asked or by default where the 64-row form would
// split K and the 16-row grid is 128..384 work-groups (measured: IQ4_XS
// 4096 x 14336 pre-quantized 8.8 us against 12.8 split four ways; Q4_K
// 4096 x 4096 4.7 against 6.8; 6144 x 4096 5.8 against 7.0; at 14336 rows,
// 896 work-groups, slower: 10.5 against 8.4). Fused quantization only up
// to 16 blocks of K: each
// work-group quantizes all of K, which at Q4_K 4096 x 14336 costs more than
// the K split saves (the decoder step 1 us slower). Its LDS (all of K
// staged) must fit.
bool narrow_form(int type, uint64_t rows, uint64_t nb, uint64_t m, bool fused, const GemvSplitK& sk, size_t& lds) {
  if (sk.narrow == 0) return false;
  if (sk.narrow < 0) {
    const uint64_t wgs = (rows + kNarrowRows - 1) / kNarrowRows;
    if (sk.ks <= 1 || wgs < 128 || wgs > 384 || (fused && nb > 16)) return false;
  }
  lds = gemv_lds_bytes(type, nb, m, 8);
  return lds <= 65536;
}

template <bool FUSED>
void launch_gemv_narrow(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, const int8_t* values,
                        const float* scales, const int32_t* sums, const float* x, uint64_t m, float* y,
                        const float* addend, uint64_t addend_stride, size_t lds, hipStream_t stream) {
  dim3 grid(static_cast<unsigned>((rows + kNarrowRows - 1) / kNarrowRows)), block(512);
  const int inb = static_cast<int>(nb);
  if (type == kTypeQ4K) {
    switch (m) {
#define X(MM)                                                                                                  \
  case MM:                                                                                                     \
    hipLaunchKernelGGL((gemv_narrow_kernel<kTypeQ4K, MM, FUSED>), grid, block, lds, stream, tiled, inb, rows,   \
                       values, scales, sums, x, y, addend, addend_stride, Fusion{});                           \
    break;
      MQ_GEMV_CASES(X)
#undef X
      default:
        break;
    }
  } else {
    switch (m) {
#define X(MM)                                                                                                    \
  case MM:                                                                                                       \
    hipLaunchKernelGGL((gemv_narrow_kernel<kTypeIq4Xs, MM, FUSED>), grid, block, lds, stream, tiled, inb, rows,   \
                       values, scales, nullptr, x, y, addend, addend_stride, Fusion{});                          \
    break;
      MQ_GEMV_CASES(X)
#undef X
      default:
        break;
    }
  }
}

// The one-block-per-wave form: rows without a K split (enough 64-row
// blocks to cover the CUs), 2..16 super-blocks, m <= 8, unless a sweep
// forces the waves per work-group. Q4_K 14336 x 4096 m = 1 fused: 8.4 ->
// 7.6 us (two blocks per wave at 8 waves against one per wave at 16).
bool wave_form(uint64_t nb, uint64_t m, int splits_hint, const GemvSplitK& sk, size_t& lds, int type) {
  if (sk.ks != 1 || m > 8 || nb < 2 || nb > 16 || splits_hint > 0 || sk.narrow == 1) return false;
  lds = gemv_lds_bytes(type, nb, m, static_cast<int>(nb));
  return lds <= 65536;
}

template <bool FUSED, int EPI = kEpiPlain, bool NORM = false>
void launch_gemv_wave(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, const int8_t* values,
                      const float* scales, const int32_t* sums, const float* x, uint64_t m, float* y,
                      const float* addend, uint64_t addend_stride, size_t lds, const Fusion& fu, hipStream_t stream) {
  dim3 grid(static_cast<unsigned>((rows + 63) / 64)), block(static_cast<unsigned>(64 * nb));
  const int inb = static_cast<int>(nb);
  if constexpr (EPI != kEpiPlain || NORM) {
    // the decode-step epilogues and the rmsnorm staging take one activation row
    if (type == kTypeQ4K)
      hipLaunchKernelGGL((gemv_wave_int8_kernel<kTypeQ4K, 1, FUSED, EPI, NORM>), grid, block, lds, stream, tiled, inb,
                         rows, x, fu.norm_w, values, scales, sums, y, addend, addend_stride, fu);
    else
      hipLaunchKernelGGL((gemv_wave_int8_kernel<kTypeIq4Xs, 1, FUSED, EPI, NORM>), grid, block, lds, stream, tiled,
                         inb, rows, x, fu.norm_w, values, scales, nullptr, y, addend, addend_stride, fu);
  } else if (type == kTypeQ4K) {
    switch (m) {
#define X(MM)                                                                                                   \
  case MM:                                                                                                      \
    hipLaunchKernelGGL((gemv_wave_int8_kernel<kTypeQ4K, MM, FUSED, EPI>), grid, block, lds, stream, tiled, inb, \
                       rows, x, fu.norm_w, values, scales, sums, y, addend, addend_stride, fu);                 \
    break;
      X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8)
#undef X
      default:
        break;
    }
  } else {
    switch (m) {
#define X(MM)                                                                                                     \
  case MM:                                                                                                        \
    hipLaunchKernelGGL((gemv_wave_int8_kernel<kTypeIq4Xs, MM, FUSED, EPI>), grid, block, lds, stream, tiled, inb, \
                       rows, x, fu.norm_w, values, scales, nullptr, y, addend, addend_stride, fu);                \
    break;
      X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8)
#undef X
      default:
        break;
    }
  }
}

template <bool FUSED>
void launch_gemv_lds(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, const int8_t* values,
                     const float* scales, const int32_t* sums, const float* x, uint64_t m, float* y,
                     const float* addend, uint64_t addend_stride, int splits, int splits_hint, const GemvSplitK& sk,
                     size_t lds, hipStream_t stream) {
  size_t narrow_lds = 0;
  if (narrow_form(type, rows, nb, m, FUSED, sk, narrow_lds)) {
    launch_gemv_narrow<FUSED>(type, tiled, rows, nb, values, scales, sums, x, m, y, addend, addend_stride,
                              narrow_lds, stream);
    return;
  }
  size_t wave_lds = 0;
  if (wave_form(nb, m, splits_hint, sk, wave_lds, type)) {
    launch_gemv_wave<FUSED>(type, tiled, rows, nb, values, scales, sums, x, m, y, addend, addend_stride, wave_lds,
                            Fusion{}, stream);
    return;
  }
  dim3 grid(static_cast<unsigned>((rows + 63) / 64), static_cast<unsigned>(sk.ks)), block(64 * splits);
  const int inb = static_cast<int>(nb);
  const SplitK k{sk.partials, sk.counters, sk.ks};
  if (type == kTypeQ4K) {
    switch (m) {
#define X(MM)                                                                                                  \
  case MM:                                                                                                     \
    hipLaunchKernelGGL((gemv_lds_int8_kernel<kTypeQ4K, MM, FUSED>), grid, block, lds, stream, tiled, inb, rows, \
                       values, scales, sums, x, y, addend, addend_stride, k, Fusion{});                        \
    break;
      MQ_GEMV_CASES(X)
#undef X
      default:
        break;
    }
  } else {
    switch (m) {
#define X(MM)                                                                                                    \
  case MM:                                                                                                       \
    hipLaunchKernelGGL((gemv_lds_int8_kernel<kTypeIq4Xs, MM, FUSED>), grid, block, lds, stream, tiled, inb, rows, \
                       values, scales, nullptr, x, y, addend, addend_stride, k, Fusion{});                       \
    break;
      MQ_GEMV_CASES(X)
#undef X
      default:
        break;
    }
  }
}

// The LDS form's launch shape, or false when its LDS would exceed 64 KiB.
bool lds_form_shape(int type, uint64_t rows, uint64_t nb, uint64_t m, int splits_hint, int ks, int& splits,
                    size_t& lds) {
  if (m < 1 || m > 8 || ks < 1) return false;
  const uint64_t nbk = (nb + ks - 1) / ks;
  splits = splits_hint;
  if (splits < 1) {
    splits = 1;
    while (splits < 8 && static_cast<uint64_t>(2 * splits) <= nbk) splits *= 2;
  }
  if (splits > lds_form_max_splits(m)) splits = lds_form_max_splits(m);
  lds = gemv_lds_bytes(type, nbk, m, splits);
  return lds <= 65536;
}

}  // namespace

GemvShape gemv_int8_shape(int type, uint64_t rows, uint64_t nb, uint64_t m, int splits, int variant,
                          const GemvSplitK& sk) {
  GemvShape g;
  int lds_splits = 0;
  size_t lds = 0;
  const bool lds_fits = lds_form_shape(type, rows, nb, m, splits, sk.ks, lds_splits, lds);
  if (variant == 0) variant = lds_fits ? 3 : (m <= 4 ? 2 : 1);
  if (variant == 3 && lds_fits) {
    size_t narrow_lds = 0;
    if (narrow_form(type, rows, nb, m, false, sk, narrow_lds)) {
      g.form = kGemvFormNarrow;
      g.waves = 8;
      g.grid_x = static_cast<unsigned>((rows + kNarrowRows - 1) / kNarrowRows);
      g.lds = narrow_lds;
      return g;
    }
    size_t wave_lds = 0;
    if (wave_form(nb, m, splits, sk, wave_lds, type)) {
      g.form = kGemvFormWave;
      g.waves = static_cast<int>(nb);
      g.grid_x = static_cast<unsigned>((rows + 63) / 64);
      g.lds = wave_lds;
      return g;
    }
    g.form = kGemvFormLds;
    g.waves = lds_splits;
    g.grid_x = static_cast<unsigned>((rows + 63) / 64);
    g.grid_y = static_cast<unsigned>(sk.ks);
    g.lds = lds;
    return g;
  }
  // Waves per work-group never exceed what each kernel is built for: the
  // other forms have launch bound 512 and 8 reduction slots.
  if (splits < 1) splits = gemv_default_splits(rows, nb, m, variant);
  g.waves = splits > 8 ? 8 : splits;
  if (variant >= 2 && m <= 4) {
    g.form = kGemvFormRows;
    g.grid_x = static_cast<unsigned>((rows + 63) / 64);
  } else {
    g.form = kGemvFormLanes8;
    g.grid_x = static_cast<unsigned>((rows + 7) / 8);
  }
  return g;
}

void launch_gemv_int8(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, const int8_t* values,
                      const float* scales, const int32_t* sums, uint64_t m, float* y, const float* addend,
                      uint64_t addend_stride, int splits, int variant, const GemvSplitK& sk,
                      hipStream_t stream) {
  const int inb = static_cast<int>(nb);
  const GemvShape g = gemv_int8_shape(type, rows, nb, m, splits, variant, sk);
  if (g.form == kGemvFormLds || g.form == kGemvFormNarrow || g.form == kGemvFormWave) {
    int lds_splits = 0;
    size_t lds = 0;
    lds_form_shape(type, rows, nb, m, splits, sk.ks, lds_splits, lds);
    launch_gemv_lds<false>(type, tiled, rows, nb, values, scales, sums, nullptr, m, y, addend, addend_stride,
                           lds_splits, splits, sk, lds, stream);
    return;
  }
  splits = g.waves;
  if (g.form == kGemvFormRows) {
    dim3 grid(g.grid_x), block(64 * splits);
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

bool launch_gemv_fused(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, const float* x, uint64_t m,
                       float* y, const float* addend, uint64_t addend_stride, int splits, const GemvSplitK& sk,
                       hipStream_t stream) {
  int lds_splits = 0;
  size_t lds = 0;
  if (!lds_form_shape(type, rows, nb, m, splits, sk.ks, lds_splits, lds)) return false;
  launch_gemv_lds<true>(type, tiled, rows, nb, nullptr, nullptr, nullptr, x, m, y, addend, addend_stride,
                        lds_splits, splits, sk, lds, stream);
  return true;
}

bool launch_gemv_decode_fused(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, const float* x, float* y,
                              bool norm, int epilogue, const GemvFusion& fu, const GemvSplitK& sk,
                              hipStream_t stream) {
  const int inb = static_cast<int>(nb);
  const int key = (type == kTypeQ4K ? 0 : 8) + (norm ? 4 : 0) + epilogue;
  size_t narrow_lds = 0;
  if (epilogue != kEpiSiluPairs && narrow_form(type, rows, nb, 1, true, sk, narrow_lds)) {
    // the same form as the plain fused GEMV of this shape takes
    dim3 grid(static_cast<unsigned>((rows + kNarrowRows - 1) / kNarrowRows)), block(512);
    switch (key) {
#define X(T, KEY, N, E)                                                                                        \
  case KEY:                                                                                                    \
    hipLaunchKernelGGL((gemv_narrow_kernel<T, 1, true, N, E>), grid, block, narrow_lds, stream, tiled, inb,     \
                       rows, nullptr, nullptr, nullptr, x, y, nullptr, 0, fu);                                 \
    return true;
      X(kTypeQ4K, 1, false, kEpiRope) X(kTypeQ4K, 4, true, kEpiPlain) X(kTypeQ4K, 5, true, kEpiRope)
      X(kTypeIq4Xs, 9, false, kEpiRope) X(kTypeIq4Xs, 12, true, kEpiPlain) X(kTypeIq4Xs, 13, true, kEpiRope)
#undef X
      default:
        return false;
    }
  }
  size_t wave_lds = 0;
  if (wave_form(nb, 1, 0, sk, wave_lds, type)) {
    // the same form as the plain fused GEMV of this shape takes (with the
    // rmsnorm: each wave's squares of its block, summed over the waves)
#define MQ_WAVE(E, N)                                                                                       \
  launch_gemv_wave<true, E, N>(type, tiled, rows, nb, nullptr, nullptr, nullptr, x, 1, y, nullptr, 0, wave_lds, \
                               fu, stream)
    if (epilogue == kEpiRope) {
      if (norm) MQ_WAVE(kEpiRope, true); else MQ_WAVE(kEpiRope, false);
    } else if (epilogue == kEpiSiluPairs) {
      if (norm) MQ_WAVE(kEpiSiluPairs, true); else MQ_WAVE(kEpiSiluPairs, false);
    } else {
      if (norm) MQ_WAVE(kEpiPlain, true); else MQ_WAVE(kEpiPlain, false);
    }
#undef MQ_WAVE
    return true;
  }
  int splits = 0;
  size_t lds = 0;
  if (!lds_form_shape(type, rows, nb, 1, 0, sk.ks, splits, lds)) return false;
  dim3 grid(static_cast<unsigned>((rows + 63) / 64), static_cast<unsigned>(sk.ks)), block(64 * splits);
  const SplitK k{sk.partials, sk.counters, sk.ks};
  switch (key) {
#define X(T, KEY, N, E)                                                                                              \
  case KEY:                                                                                                          \
    hipLaunchKernelGGL((gemv_lds_int8_kernel<T, 1, true, N, E>), grid, block, lds, stream, tiled, inb, rows, nullptr, \
                       nullptr, nullptr, x, y, nullptr, 0, k, fu);                                                    \
    return true;
    X(kTypeQ4K, 1, false, kEpiRope) X(kTypeQ4K, 2, false, kEpiSiluPairs) X(kTypeQ4K, 4, true, kEpiPlain)
    X(kTypeQ4K, 5, true, kEpiRope) X(kTypeQ4K, 6, true, kEpiSiluPairs)
    X(kTypeIq4Xs, 9, false, kEpiRope) X(kTypeIq4Xs, 10, false, kEpiSiluPairs) X(kTypeIq4Xs, 12, true, kEpiPlain)
    X(kTypeIq4Xs, 13, true, kEpiRope) X(kTypeIq4Xs, 14, true, kEpiSiluPairs)
#undef X
    default:
      return false;
  }
}

// ---- embedding and input-major products (any format) --------------------------

#define MQ_ALL_TYPES(X) X(kTypeQ4K) X(kTypeIq4Xs) X(kTypeQ8_0) X(kTypeQ4_0) X(kTypeIq4Nl) X(kTypeQ2K) X(kTypeQ3K) X(kTypeQ5K) X(kTypeQ6K)
#define MQ_GRID_TYPES(X) X(kTypeIq2Xxs) X(kTypeIq2Xs) X(kTypeIq2S) X(kTypeIq3Xxs) X(kTypeIq3S)
#define MQ_TABLE_TYPES(X) MQ_ALL_TYPES(X) MQ_GRID_TYPES(X)

void launch_embedding(int type, const uint8_t* tiled, uint64_t nb, int transposed, const uint32_t* ids,
                      uint64_t count, uint64_t dim, float scale, int scaled, float* out, hipStream_t stream) {
  const uint64_t threads = transposed ? count * dim : count * (dim / 32);
  switch (type) {
#define X(T)                                                                                                       \
  case T:                                                                                                          \
    if (transposed)                                                                                                \
      hipLaunchKernelGGL(embed_columns_kernel<T>, dim3(grid_for(threads, 256)), dim3(256), 0, stream, tiled, nb,   \
                         ids, count, dim, scale, scaled, out);                                                     \
    else                                                                                                           \
      hipLaunchKernelGGL(embed_rows_kernel<T>, dim3(grid_for(threads, 256)), dim3(256), 0, stream, tiled, nb, ids, \
                         count, dim, scale, scaled, out);                                                          \
    break;
    MQ_TABLE_TYPES(X)
#undef X
    default:
      break;
  }
}

int axpy_ksplit(uint64_t k, uint64_t n) {
  // about 64K threads in flight: (n / 16) per split
  const uint64_t per = n / 16 ? n / 16 : 1;
  uint64_t ks = (65536 + per - 1) / per;
  if (ks > k) ks = k;
  if (ks > 256) ks = 256;
  return static_cast<int>(ks < 1 ? 1 : ks);
}

void launch_axpy(int type, const uint8_t* tiled, uint64_t nb, uint64_t k, uint64_t n, const float* x, uint64_t m,
                 float* y, const float* addend, uint64_t addend_stride, float* part, int ks, hipStream_t stream) {
  constexpr int MM = 4;
  const uint64_t kchunk = (k + ks - 1) / ks;
  dim3 grid(grid_for(n / 16, 256), static_cast<unsigned>(ks));
  for (uint64_t r0 = 0; r0 < m; r0 += MM) {
    const int rows = static_cast<int>(m - r0 < MM ? m - r0 : MM);
    switch (type) {
#define X(T)                                                                                                        \
  case T:                                                                                                           \
    hipLaunchKernelGGL((axpy_kernel<T, MM>), grid, dim3(256), 0, stream, tiled, nb, k, n, x + r0 * k, rows, kchunk, \
                       part);                                                                                       \
    break;
      MQ_TABLE_TYPES(X)
#undef X
      default:
        break;
    }
    hipLaunchKernelGGL(axpy_finish_kernel, dim3(grid_for(rows * n, 256)), dim3(256), 0, stream, part, ks, MM, rows, n,
                       y + r0 * n, addend ? addend + (addend_stride ? r0 * addend_stride : 0) : nullptr,
                       addend_stride);
  }
}

// ---- IQ2 / IQ3 grid formats ---------------------------------------------------

hipError_t grid_tables_upload(const uint8_t* host, hipStream_t stream) {
  hipError_t e = hipMemcpyToSymbolAsync(HIP_SYMBOL(g_iq_grids), host, kGridTableBytes, 0, hipMemcpyHostToDevice,
                                        stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  return e;
}

void launch_dequantize_grid(int type, const uint8_t* w, uint64_t rows, uint64_t nb, int logical, float* out,
                            hipStream_t stream) {
  const uint64_t threads = rows * nb * 8;
  switch (type) {
#define X(T)                                                                                                   \
  case T:                                                                                                      \
    hipLaunchKernelGGL(dequantize_grid_kernel<T>, dim3(grid_for(threads, 256)), dim3(256), 0, stream, w, rows, \
                       nb, logical, out);                                                                      \
    break;
    MQ_GRID_TYPES(X)
#undef X
    default:
      break;
  }
}

void launch_gemv_grid(int type, const uint8_t* w, uint64_t nb, uint64_t rows, const int8_t* xv, const float* xs,
                      const float* xf, uint64_t m, int int8, float* y, const float* addend, uint64_t addend_stride,
                      hipStream_t stream) {
  // at most 4 work-groups per CU: each copies the format's grid table once
  // (and the int8 activations, when table and activations fit 64 KiB)
  const uint64_t wgs = (rows + kGridGemvWaves - 1) / kGridGemvWaves;
  const dim3 grid(static_cast<unsigned>(wgs < 1024 ? wgs : 1024)), block(64 * kGridGemvWaves);
  const uint64_t table = static_cast<uint64_t>(grid_table_size(type)) + kGridSignTableBytes;
  const uint64_t staged = table + m * nb * 256 + 4 * m * nb * 8;
  const bool stage = int8 && staged <= 65536;
  switch (type) {
#define MQ_GRID_M(T, MM)                                                                                             \
  case MM:                                                                                                           \
    if (stage)                                                                                                       \
      hipLaunchKernelGGL((gemv_grid_kernel<T, MM, true, true>), grid, block, staged, stream, w, nb, rows, xv, xs, xf, \
                         y, addend, addend_stride);                                                                  \
    else if (int8)                                                                                                   \
      hipLaunchKernelGGL((gemv_grid_kernel<T, MM, true, false>), grid, block, table, stream, w, nb, rows, xv, xs, xf, \
                         y, addend, addend_stride);                                                                  \
    else                                                                                                             \
      hipLaunchKernelGGL((gemv_grid_kernel<T, MM, false, false>), grid, block, table, stream, w, nb, rows, xv, xs,   \
                         xf, y, addend, addend_stride);                                                              \
    break;
#define X(T)                                                                                                 \
  case T:                                                                                                    \
    switch (m) {                                                                                             \
      MQ_GRID_M(T, 1) MQ_GRID_M(T, 2) MQ_GRID_M(T, 3) MQ_GRID_M(T, 4) MQ_GRID_M(T, 5) MQ_GRID_M(T, 6)        \
      MQ_GRID_M(T, 7) MQ_GRID_M(T, 8)                                                                        \
      default:                                                                                               \
        break;                                                                                               \
    }                                                                                                        \
    break;
    MQ_GRID_TYPES(X)
#undef X
#undef MQ_GRID_M
    default:
      break;
  }
}

// ---- plane formats ----------------------------------------------------------

void launch_repack_planes(int type, const uint8_t* raw, uint64_t rows, uint64_t k, uint64_t nb, uint8_t* tiled,
                          hipStream_t stream) {
  const uint64_t threads = rows * nb * (plane_count(type) + (plane_shared_width(type) ? 1 : 0));
  switch (type) {
#define X(T)                                                                                                 \
  case T:                                                                                                    \
    hipLaunchKernelGGL(repack_planes_kernel<T>, dim3(grid_for(threads, 256)), dim3(256), 0, stream, raw, rows, \
                       k, nb, tiled);                                                                        \
    break;
    X(kTypeQ8_0) X(kTypeQ4_0) X(kTypeIq4Nl) X(kTypeQ2K) X(kTypeQ3K) X(kTypeQ5K) X(kTypeQ6K)
#undef X
    default:
      break;
  }
}

void launch_dequantize_planes(int type, const uint8_t* tiled, uint64_t rows, uint64_t k, uint64_t nb, int logical,
                              float* out, hipStream_t stream) {
  const uint64_t threads = rows * (k / 32);
  switch (type) {
#define X(T)                                                                                                        \
  case T:                                                                                                           \
    hipLaunchKernelGGL(dequantize_planes_kernel<T>, dim3(grid_for(threads, 256)), dim3(256), 0, stream, tiled, rows, \
                       k, nb, logical, out);                                                                        \
    break;
    X(kTypeQ8_0) X(kTypeQ4_0) X(kTypeIq4Nl) X(kTypeQ2K) X(kTypeQ3K) X(kTypeQ5K) X(kTypeQ6K)
#undef X
    default:
      break;
  }
}

namespace {

// LDS of the plane GEMV: int8 values [m][kn] and a 16-byte record per run,
// or the cross-wave reduction, whichever is larger.
size_t gemv_planes_lds_bytes(uint64_t nbk, uint64_t m, int splits) {
  const size_t act = m * nbk * 256 + m * nbk * 8 * 16;
  const size_t red = static_cast<size_t>(splits) * m * 2 * 64 * 4;
  return act > red ? act : red;
}

int planes_waves(uint64_t nbk, int hint) {
  int splits = hint;
  if (splits < 1) {
    splits = 1;
    while (splits < 8 && static_cast<uint64_t>(2 * splits) <= nbk) splits *= 2;
  }
  return splits > 8 ? 8 : splits;  // launch bound 512
}

}  // namespace

int gemv_planes_min_ksplit(uint64_t nb, uint64_t m) {
  int ks = 1;
  while (gemv_planes_lds_bytes((nb + ks - 1) / ks, m, 8) > 65536 && static_cast<uint64_t>(ks) < nb) ++ks;
  return ks;
}

void launch_gemv_planes_int8(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, uint64_t k,
                             const int8_t* values, const float* scales, const int32_t* sums, const float* x,
                             uint64_t m, float* y, const float* addend, uint64_t addend_stride, int splits,
                             const GemvSplitK& sk, hipStream_t stream) {
  const uint64_t nbk = (nb + sk.ks - 1) / sk.ks;
  const int waves = planes_waves(nbk, splits);
  const size_t lds = gemv_planes_lds_bytes(nbk, m, waves);
  dim3 grid(static_cast<unsigned>((rows + 63) / 64), static_cast<unsigned>(sk.ks)), block(64 * waves);
  const int inb = static_cast<int>(nb);
  const SplitK kk{sk.partials, sk.counters, sk.ks};
  const int key = type * 16 + static_cast<int>(m) - 1;
  switch (key) {
#define Y(T, MM)                                                                                                  \
  case T * 16 + MM - 1:                                                                                           \
    if (x)                                                                                                        \
      hipLaunchKernelGGL((gemv_planes_int8_kernel<T, MM, true>), grid, block, lds, stream, tiled, inb, rows, k,    \
                         values, scales, sums, x, y, addend, addend_stride, kk);                                  \
    else                                                                                                          \
      hipLaunchKernelGGL((gemv_planes_int8_kernel<T, MM, false>), grid, block, lds, stream, tiled, inb, rows, k,   \
                         values, scales, sums, x, y, addend, addend_stride, kk);                                  \
    break;
#define X(T) Y(T, 1) Y(T, 2) Y(T, 3) Y(T, 4) Y(T, 5) Y(T, 6) Y(T, 7) Y(T, 8)
    X(kTypeQ8_0) X(kTypeQ4_0) X(kTypeIq4Nl) X(kTypeQ2K) X(kTypeQ3K) X(kTypeQ5K) X(kTypeQ6K)
#undef X
#undef Y
    default:
      break;
  }
}

void launch_gemv_planes_f32(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, uint64_t k, const float* x,
                            uint64_t m, float* y, const float* addend, uint64_t addend_stride, int splits,
                            hipStream_t stream) {
  const int waves = planes_waves(nb, splits);
  const size_t lds = static_cast<size_t>(waves) * m * 2 * 64 * 4;
  dim3 grid(static_cast<unsigned>((rows + 63) / 64)), block(64 * waves);
  const int inb = static_cast<int>(nb);
  const int key = type * 16 + static_cast<int>(m) - 1;
  switch (key) {
#define Y(T, MM)                                                                                                   \
  case T * 16 + MM - 1:                                                                                            \
    hipLaunchKernelGGL((gemv_planes_f32_kernel<T, MM>), grid, block, lds, stream, tiled, inb, rows, k, x, y, addend, \
                       addend_stride);                                                                             \
    break;
#define X(T) Y(T, 1) Y(T, 2) Y(T, 3) Y(T, 4) Y(T, 5) Y(T, 6) Y(T, 7) Y(T, 8)
    X(kTypeQ8_0) X(kTypeQ4_0) X(kTypeIq4Nl) X(kTypeQ2K) X(kTypeQ3K) X(kTypeQ5K) X(kTypeQ6K)
#undef X
#undef Y
    default:
      break;
  }
}

// K-splits for the LDS form: only when the row blocks alone leave most of
// the 256 CUs idle (4096 rows: 64 blocks -> 4 splits; 14336 rows: 224
// blocks -> none, where the split-K epilogue costs more than the last 32
// CUs would bring), and at most 4: each work-group's chain of activation
// staging, barrier, partial stores and ticket is a fixed latency, and
// measured at 1024 x 4096, 4 splits take 6.9 us where 16 take 12.0 us.
int gemv_default_ksplit(uint64_t rows, uint64_t nb) {
  const uint64_t blocks = (rows + 63) / 64;
  int ks = 1;
  while (blocks * 2 * ks <= 320 && static_cast<uint64_t>(2 * ks) <= nb && ks < 4) ks *= 2;
  return ks;
}

void launch_gemv_f32(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, const float* x, uint64_t m,
                     float* y, const float* addend, uint64_t addend_stride, int splits, hipStream_t stream) {
  splits = splits < 1 ? 1 : splits > 8 ? 8 : splits;  // launch bound 512, 8 reduction slots
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
                    float* y, const float* addend, uint64_t addend_stride, F16Range rg, hipStream_t stream,
                    int ks = 1) {
  const uint64_t rows_padded = (rows + 7) / 8 * 8;
  const uint64_t bn = 4 * NF * 16, bm = MF * 16;
  dim3 grid(static_cast<unsigned>((rows + bn - 1) / bn), static_cast<unsigned>((m + bm - 1) / bm),
            static_cast<unsigned>(ks));
  switch (type) {
#define X(T)                                                                                                     \
  case T:                                                                                                        \
    hipLaunchKernelGGL((gemm_rb_kernel<T, MF, NF>), grid, dim3(256), 0, stream, tiled, static_cast<int>(nb), rows, \
                       rows_padded, a16, m, y, addend, addend_stride, rg);                                      \
    break;
    MQ_ALL_TYPES(X)
#undef X
    default:
      break;
  }
}

template <int MF, int NF>
void launch_gemm_grid(int type, const uint8_t* w, uint64_t rows, uint64_t nb, const uint16_t* a16, uint64_t m,
                      float* y, const float* addend, uint64_t addend_stride, F16Range rg, hipStream_t stream,
                      int ks = 1) {
  const uint64_t bn = 4 * NF * 16, bm = MF * 16;
  dim3 grid(static_cast<unsigned>((rows + bn - 1) / bn), static_cast<unsigned>((m + bm - 1) / bm),
            static_cast<unsigned>(ks));
  switch (type) {
#define X(T)                                                                                                    \
  case T:                                                                                                       \
    hipLaunchKernelGGL((gemm_grid_kernel<T, MF, NF>), grid, dim3(256), 0, stream, w, static_cast<int>(nb), rows, \
                       a16, m, y, addend, addend_stride, rg);                                                  \
    break;
    MQ_GRID_TYPES(X)
#undef X
    default:
      break;
  }
}

uint64_t tiles(uint64_t rows, uint64_t m, uint64_t bn, uint64_t bm) {
  return ((rows + bn - 1) / bn) * ((m + bm - 1) / bm);
}

// Split-K sum of the register-B GEMM: y = partials of split 0 + split 1 +
// ... in split order, then + addend (the epilogue's order).
__global__ void gemm_split_reduce_kernel(const float* __restrict__ part, int ks, uint64_t m_rows, uint64_t rows,
                                         float* __restrict__ y, const float* __restrict__ addend,
                                         uint64_t addend_stride) {
  const uint64_t count = m_rows * rows;
  const uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
  if (i >= count) return;
  float v = part[i];
  for (int z = 1; z < ks; ++z) v = v + part[static_cast<uint64_t>(z) * count + i];
  if (addend) v = v + addend[(i / rows) * addend_stride + i % rows];
  y[i] = v;
}

}  // namespace

// The K-split form's split count over work-groups: 1 once its 128 x 256
// tiles cover most CUs, else enough splits for about 224 work-groups, each
// with at least two super-blocks (one per K half).
uint64_t ks_form_splits(uint64_t rows, uint64_t m, uint64_t nb) {
  const uint64_t t = tiles(rows, m, kKsBN, kKsBM);
  if (t >= 160) return 1;
  uint64_t z = (224 + t - 1) / t;
  if (z > nb / 2) z = nb / 2;
  return z < 1 ? 1 : z;
}

int gemm_default_variant(int type, uint64_t rows, uint64_t m, uint64_t nb) {
  // Q4_K: the K-split form while it (split over work-groups if need be)
  // covers at least half the CUs: M = 128 x 14336 x 4096 39.0 us against
  // 44.2 for the split register-B form, M = 512 x 4096 x 4096 41.0 against
  // 45.6; M = 128 x 4096 x 4096 (128 work-groups of two super-blocks each)
  // 18.6 + 3.9 us (partials, then their sum) against 28.6
  if (type == kTypeQ4K) {
    const uint64_t t = tiles(rows, m, kKsBN, kKsBM);
    if (t >= 160 || t * ks_form_splits(rows, m, nb) >= 128) return 5;
  }
  // Register-B 128 x 128 tiles (two work-groups per CU fit, 2 waves per
  // SIMD); the 128 x 256 tile only once there are work-groups for every CU
  // several times over.
  if (tiles(rows, m, 256, 128) >= 1024) return 2;
  return 3;
}

// The register-B form's split-K factor: 1 unless its tiles leave most CUs
// idle (fewer than 192 work-groups); then enough splits for about 224
// work-groups, at most 8 (16 for rows of 32 or more super-blocks) and at
// most one per super-block.
int gemm_splits(int type, uint64_t rows, uint64_t m, uint64_t nb, uint64_t k, int variant) {
  if (is_plane_format(type) && k % 256 != 0) return 1;
  if (is_grid_format(type))
    variant = variant == 2 || (variant == 0 && tiles(rows, m, 256, 128) >= 1024) ? 2 : 3;
  else if (variant == 0)
    variant = gemm_default_variant(type, rows, m, nb);
  if (variant == 5 && type != kTypeQ4K) variant = 3;
  if (variant == 5) return static_cast<int>(ks_form_splits(rows, m, nb));
  if (variant != 2 && variant != 3 && variant != 4) return 1;
  const uint64_t t = tiles(rows, m, variant == 3 ? 128 : 256, variant == 4 ? 64 : 128);
  if (t >= 192) return 1;
  uint64_t ks = (224 + t - 1) / t;
  if (ks > 8) ks = 8;
  // long rows (K >= 8192) take twice the splits: the extra partials cost
  // less than the latency of the longer K range (measured: IQ4_XS
  // 4096 x 14336 at M = 512 134.7 us with 2 splits, 118.6 us with 4; at
  // 16 super-blocks more splits than this lost: 14336 x 4096 at M = 128
  // 46.0 us with 2, 54.0 us with 5)
  if (nb >= 32) ks *= 2;
  if (ks > nb) ks = nb;
  return static_cast<int>(ks);
}

void launch_gemm(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, uint64_t k, const uint16_t* a16,
                 uint64_t m, float* y, const float* addend, uint64_t addend_stride, int variant,
                 hipStream_t stream, F16Range rg, float* part) {
  const int ks = part ? gemm_splits(type, rows, m, nb, k, variant) : 1;
  if (ks > 1 && is_grid_format(type)) {
    if (variant == 2)
      launch_gemm_grid<8, 4>(type, tiled, rows, nb, a16, m, part, nullptr, 0, rg, stream, ks);
    else
      launch_gemm_grid<8, 2>(type, tiled, rows, nb, a16, m, part, nullptr, 0, rg, stream, ks);
    hipLaunchKernelGGL(gemm_split_reduce_kernel, dim3(grid_for(m * rows, 256)), dim3(256), 0, stream, part, ks, m,
                       rows, y, addend, addend_stride);
    return;
  }
  if (ks > 1 && type == kTypeQ4K && (variant == 5 || (variant == 0 && gemm_default_variant(type, rows, m, nb) == 5))) {
    // the K-split form over ks K ranges into `part`, then their sum
    const uint64_t rows_padded = (rows + 7) / 8 * 8;
    dim3 ks_grid(static_cast<unsigned>((rows + kKsBN - 1) / kKsBN), static_cast<unsigned>((m + kKsBM - 1) / kKsBM),
                 static_cast<unsigned>(ks));
    hipLaunchKernelGGL(gemm_ks_kernel, ks_grid, dim3(kKsThreads), 0, stream, tiled, static_cast<int>(nb), rows,
                       rows_padded, a16, m, part, nullptr, 0, rg);
    hipLaunchKernelGGL(gemm_split_reduce_kernel, dim3(grid_for(m * rows, 256)), dim3(256), 0, stream, part, ks, m,
                       rows, y, addend, addend_stride);
    return;
  }
  if (ks > 1) {
    // the register-B form over ks K ranges into `part`, then their sum
    const int v = variant == 0 ? gemm_default_variant(type, rows, m, nb) : (variant == 5 ? 3 : variant);
    if (v == 2)
      launch_gemm_rb<8, 4>(type, tiled, rows, nb, a16, m, part, nullptr, 0, rg, stream, ks);
    else if (v == 4)
      launch_gemm_rb<4, 4>(type, tiled, rows, nb, a16, m, part, nullptr, 0, rg, stream, ks);
    else
      launch_gemm_rb<8, 2>(type, tiled, rows, nb, a16, m, part, nullptr, 0, rg, stream, ks);
    hipLaunchKernelGGL(gemm_split_reduce_kernel, dim3(grid_for(m * rows, 256)), dim3(256), 0, stream, part, ks, m,
                       rows, y, addend, addend_stride);
    return;
  }
  const uint64_t rows_padded = (rows + 7) / 8 * 8;
  dim3 grid(static_cast<unsigned>((rows + kBN - 1) / kBN), static_cast<unsigned>((m + kBM - 1) / kBM));
  if (is_grid_format(type)) {
    // grid formats: raw blocks, whole super-blocks (k % 256 == 0)
    if (variant == 0) variant = tiles(rows, m, 256, 128) >= 1024 ? 2 : 3;
    if (variant == 2)
      launch_gemm_grid<8, 4>(type, tiled, rows, nb, a16, m, y, addend, addend_stride, rg, stream);
    else
      launch_gemm_grid<8, 2>(type, tiled, rows, nb, a16, m, y, addend, addend_stride, rg, stream);
    return;
  }
  // plane formats whose rows end inside a group take the LDS-B form
  if (is_plane_format(type) && k % 256 != 0) variant = 1;
  if (variant == 1 && is_plane_format(type)) {
    switch (type) {
#define X(T)                                                                                                       \
  case T:                                                                                                          \
    hipLaunchKernelGGL(gemm_kernel<T>, grid, dim3(256), 0, stream, tiled, static_cast<int>(nb), rows, rows_padded, \
                       a16, m, y, addend, addend_stride, k, rg);                                                   \
    return;
      X(kTypeQ8_0) X(kTypeQ4_0) X(kTypeIq4Nl) X(kTypeQ2K) X(kTypeQ3K) X(kTypeQ5K) X(kTypeQ6K)
#undef X
      default:
        return;
    }
  }
  if (variant == 0) variant = gemm_default_variant(type, rows, m, nb);
  if (variant == 5 && type != kTypeQ4K) variant = 3;
  switch (variant) {
    case 5: {
      dim3 ks_grid(static_cast<unsigned>((rows + kKsBN - 1) / kKsBN), static_cast<unsigned>((m + kKsBM - 1) / kKsBM));
      hipLaunchKernelGGL(gemm_ks_kernel, ks_grid, dim3(kKsThreads), 0, stream, tiled, static_cast<int>(nb), rows,
                         rows_padded, a16, m, y, addend, addend_stride, rg);
      return;
    }
    case 2:
      launch_gemm_rb<8, 4>(type, tiled, rows, nb, a16, m, y, addend, addend_stride, rg, stream);
      return;
    case 3:
      launch_gemm_rb<8, 2>(type, tiled, rows, nb, a16, m, y, addend, addend_stride, rg, stream);
      return;
    case 4:
      launch_gemm_rb<4, 4>(type, tiled, rows, nb, a16, m, y, addend, addend_stride, rg, stream);
      return;
    default:
      break;
  }
  if (type == kTypeQ4K)
    hipLaunchKernelGGL(gemm_kernel<kTypeQ4K>, grid, dim3(256), 0, stream, tiled, static_cast<int>(nb), rows,
                       rows_padded, a16, m, y, addend, addend_stride, k, rg);
  else
    hipLaunchKernelGGL(gemm_kernel<kTypeIq4Xs>, grid, dim3(256), 0, stream, tiled, static_cast<int>(nb), rows,
                       rows_padded, a16, m, y, addend, addend_stride, k, rg);
}

}  // namespace mq
