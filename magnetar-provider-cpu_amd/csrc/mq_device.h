// Device-side layout and decode helpers shared by the gfx950 kernels.
//
// HBM layout of a packed weight (chosen at upload; the bytes are the
// checkpoint's own, permuted, never re-encoded):
//
//   stored rows are grouped by 8 (a "row group", zero-padded to a multiple
//   of 8 rows); each (row group g, super-block b) is one contiguous tile.
//
//   Q4_K tile (1152 B): 9 planes x 8 rows x 16 B. Plane 0 holds each row's
//     block bytes 0..15 (d, dmin, scales[12]); plane 1+p holds block bytes
//     16+16p .. 31+16p (the quants).
//   IQ4_XS tile (1088 B): 8 rows x 8 B of block bytes 0..7 (d, scales_h,
//     scales_l[4]), then 8 planes x 8 rows x 16 B, plane p holding block
//     bytes 8+16p .. 23+16p (run p's 32 indices).
//
//   Plane formats (Q8_0, Q4_0, IQ4_NL, Q5_K, Q6_K): a "group" is 256
//     values of a row (a K-quant super-block, or eight 32-value blocks);
//     the tile is kPlanes planes x 8 rows x 16 B, plane p of row r at
//     128 p + 16 r, plus for Q6_K one shared 16-byte plane holding the 8
//     rows' f16 d (row r at byte 2 r):
//       Q8_0   17 planes: 0 = the 8 blocks' f16 d; 1 + 2i + h = block i's
//              quants 16h .. 16h + 15.
//       Q4_0, IQ4_NL  9 planes: 0 = the 8 blocks' f16 d; 1 + i = block i's
//              16 nibble-pair bytes.
//       Q5_K   11 planes: the super-block's bytes 16p .. 16p + 15 (0: d,
//              dmin, scales; 1-2: high bits; 3-10: nibbles).
//       Q6_K   13 planes: bytes 16p .. 16p + 15 (0-7: low nibbles, 8-11:
//              high bits, 12: the 16 i8 scales), then the shared d plane.
//       Q2_K   5 planes: bytes 16p .. 16p + 15 (0: the 16 scale/min bytes,
//              1-4: the 2-bit quants), then a shared 32-byte region with
//              each row's d and dmin (row r at byte 4 r).
//       Q3_K   7 planes: bytes 16p .. 16p + 15 (0-1: high-bit mask, 2-5:
//              the 2-bit quants, 6: the 12 scale bytes and d, 2 bytes pad).
//     A row whose K is not a multiple of 256 (32-value formats) ends in a
//     group padded with zero blocks (d = 0).
//
//   tile(g, b) starts at (g * nb + b) * tile_bytes, nb = ceil(K / 256).
//
// So a 64-lane load of one plane by 8 rows x 8 blocks touches eight whole
// 128-byte lines, and a GEMM K-step reads whole lines per 8 rows.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mq {

constexpr int kTypeQ4K = 12;
constexpr int kTypeIq4Xs = 23;
constexpr int kGroupRows = 8;
constexpr int kQ4kBlockBytes = 144;
constexpr int kIq4xsBlockBytes = 136;
constexpr int kQ4kTileBytes = 1152;
constexpr int kIq4xsTileBytes = 1088;

constexpr int kTypeQ4_0 = 2;
constexpr int kTypeQ8_0 = 8;
constexpr int kTypeQ2K = 10;
constexpr int kTypeQ3K = 11;
constexpr int kTypeQ5K = 13;
constexpr int kTypeQ6K = 14;
constexpr int kTypeIq4Nl = 20;

// IQ2 / IQ3 grid formats: the weight keeps the checkpoint's block order
// (stored row after stored row, nb blocks each); their decode reads the
// grid tables the caller supplies once per device.
constexpr int kTypeIq2Xxs = 16;
constexpr int kTypeIq2Xs = 17;
constexpr int kTypeIq3Xxs = 18;
constexpr int kTypeIq3S = 21;
constexpr int kTypeIq2S = 22;

__host__ __device__ constexpr bool is_grid_format(int type) {
  return type == kTypeIq2Xxs || type == kTypeIq2Xs || type == kTypeIq2S || type == kTypeIq3Xxs || type == kTypeIq3S;
}

// Byte offsets of each grid table in the device copy: IQ2_XXS 256, IQ2_XS
// 512 and IQ2_S 1024 entries of 8 magnitudes, IQ3_XXS 256 and IQ3_S 512
// entries of 4.
constexpr int kGridIq2Xxs = 0, kGridIq2Xs = 2048, kGridIq2S = 6144, kGridIq3Xxs = 14336, kGridIq3S = 15360;
constexpr int kGridTableBytes = 17408;

__host__ __device__ constexpr bool is_plane_format(int type) {
  return type == kTypeQ8_0 || type == kTypeQ4_0 || type == kTypeIq4Nl || type == kTypeQ5K || type == kTypeQ6K ||
         type == kTypeQ2K || type == kTypeQ3K;
}

// Per-row 16-byte planes of a plane format's tile (shared region apart).
__host__ __device__ constexpr int plane_count(int type) {
  return type == kTypeQ8_0                          ? 17
         : (type == kTypeQ4_0 || type == kTypeIq4Nl) ? 9
         : type == kTypeQ5K                          ? 11
         : type == kTypeQ2K                          ? 5
         : type == kTypeQ3K                          ? 7
                                                     : 13;
}

// Bytes per row of the tile's shared region after the planes: Q6_K's d,
// Q2_K's d and dmin.
__host__ __device__ constexpr int plane_shared_width(int type) {
  return type == kTypeQ6K ? 2 : type == kTypeQ2K ? 4 : 0;
}

__host__ __device__ constexpr bool plane_shared_d(int type) { return plane_shared_width(type) != 0; }

// Checkpoint block geometry: values and bytes per block.
__host__ __device__ constexpr int block_values(int type) {
  return (type == kTypeQ8_0 || type == kTypeQ4_0 || type == kTypeIq4Nl) ? 32 : 256;
}

__host__ __device__ constexpr int block_bytes_of(int type) {
  return type == kTypeQ8_0 ? 34
         : (type == kTypeQ4_0 || type == kTypeIq4Nl) ? 18
         : type == kTypeQ4K ? kQ4kBlockBytes
         : type == kTypeQ5K ? 176
         : type == kTypeQ6K ? 210
         : type == kTypeQ2K ? 84
         : type == kTypeQ3K ? 110
         : type == kTypeIq2Xxs ? 66
         : type == kTypeIq2Xs ? 74
         : type == kTypeIq2S ? 82
         : type == kTypeIq3Xxs ? 98
         : type == kTypeIq3S ? 110
         : kIq4xsBlockBytes;
}

__host__ __device__ constexpr int tile_bytes(int type) {
  return type == kTypeQ4K     ? kQ4kTileBytes
         : type == kTypeIq4Xs ? kIq4xsTileBytes
                              : 128 * plane_count(type) + 8 * plane_shared_width(type);
}

// The GGUF kvalues_iq4nl codebook packed 4 bytes per word (little end
// first): words 0..3 hold entries 0..3, 4..7, 8..11, 12..15.
constexpr uint32_t kIq4Word0 = 0xBFAD9881u;  // -127 -104 -83 -65
constexpr uint32_t kIq4Word1 = 0xF6EADDCFu;  //  -49  -35 -22 -10
constexpr uint32_t kIq4Word2 = 0x26190D01u;  //    1   13  25  38
constexpr uint32_t kIq4Word3 = 0x71594535u;  //   53   69  89 113

__device__ inline float half_bits(uint32_t bits16) {
  return __half2float(__ushort_as_half(static_cast<unsigned short>(bits16 & 0xFFFFu)));
}

// Q4_K super-block scales: run j's 6-bit scale and min (ggml
// get_scale_min_k4) from the 12 scale bytes in header words y, z, w.
// Bytes 0..3 of the result hold runs 0..3 (lo) or 4..7 (hi).
struct Q4kSixBit {
  uint32_t sc_lo, sc_hi, m_lo, m_hi;
};

__device__ inline Q4kSixBit q4k_six_bit(uint4 hdr) {
  Q4kSixBit r;
  r.sc_lo = hdr.y & 0x3F3F3F3Fu;
  r.m_lo = hdr.z & 0x3F3F3F3Fu;
  r.sc_hi = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
  r.m_hi = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
  return r;
}

__device__ inline uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }

// Run j's 6-bit scale and min as integers, j in 0..7.
__device__ inline void q4k_sc_m(const Q4kSixBit& s, int j, uint32_t& sc, uint32_t& m) {
  if (j < 4) {
    sc = byte_of(s.sc_lo, j);
    m = byte_of(s.m_lo, j);
  } else {
    sc = byte_of(s.sc_hi, j - 4);
    m = byte_of(s.m_hi, j - 4);
  }
}

// IQ4_XS run j's signed scale (ls - 32) from header words x (d | scales_h)
// and y (scales_l[4]).
__device__ inline int iq4xs_ls(uint2 hdr, int j) {
  uint32_t low = (hdr.y >> (4 * j)) & 0xFu;
  uint32_t high = (hdr.x >> (16 + 2 * j)) & 3u;
  return static_cast<int>(low | (high << 4)) - 32;
}

// Four codebook lookups: bytes of `nib` are indices 0..15, result bytes are
// the signed codebook values.
__device__ inline uint32_t iq4_lookup4(uint32_t nib) {
  uint32_t i7 = nib & 0x07070707u;
  uint32_t lo = __builtin_amdgcn_perm(kIq4Word1, kIq4Word0, i7);
  uint32_t hi = __builtin_amdgcn_perm(kIq4Word3, kIq4Word2, i7);
  uint32_t mask = ((nib >> 3) & 0x01010101u) * 0xFFu;
  return (hi & mask) | (lo & ~mask);
}

__device__ inline int sdot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// Raw buffer loads (MUBUF) over a wave-uniform base: an offset at or past
// `bytes` reads zeros without a memory access. Kernels use this to issue a
// fixed sequence of loads on every path (predicating by offset instead of
// branching), which keeps the compiler's vmcnt waits exact.
constexpr uint32_t kBufferDword3 = 0x00020000u;  // gfx9 raw buffer: 32-bit data format
constexpr uint32_t kBufferNone = 0x80000000u;    // an offset past every resource this code builds

__device__ inline __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           static_cast<int>(kBufferDword3));
}

__device__ inline uint4 buffer_ld16(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(offset), 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ inline uint32_t buffer_ld4(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
  return static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(offset), 0, 0));
}

__device__ inline uint2 buffer_ld8(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(offset), 0, 0);
  return make_uint2(v.x, v.y);
}

}  // namespace mq
