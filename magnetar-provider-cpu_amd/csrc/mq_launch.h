// Host launchers for the gfx950 kernels (defined in the .hip files).
// Every launcher checks nothing: the C-ABI layer validates shapes, buffer
// sizes and grids before calling, and reports errors to the caller.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mq {

// Raw checkpoint bytes (rows x nb blocks, row-major) -> tiled layout.
void launch_repack(int type, const uint8_t* raw, uint64_t rows, uint64_t nb,
                   uint8_t* tiled, hipStream_t stream);

// Bit-exact dequantization; logical != 0 writes out[k * rows + n] (the
// transposed, logical [K, N] view), else out[n * K + k] (stored view).
void launch_dequantize(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb,
                       int logical, float* out, hipStream_t stream);

// Int8 activation quantization of x[m][k] per 32-value block (k % 32 == 0).
void launch_quantize_activations(const float* x, uint64_t m, uint64_t k, int8_t* values,
                                 float* scales, int32_t* sums, hipStream_t stream);

// The prefill GEMM's activation operand: a16[m][k] = f16(v * 2^e_r), v =
// the int8 round trip q d of x (int8 != 0) or x itself, with e_r the power
// of two that puts row r's largest magnitude in [2^14, 2^15) (0 for rows of
// zeros or with an infinity), and row_factor[r] = 2^-e_r. k % 32 == 0.
void launch_activations_f16(const float* x, uint64_t m, uint64_t k, int int8, uint16_t* a16,
                            float* row_factor, hipStream_t stream);

// The power of two 2^f that puts a weight's largest dequantized magnitude
// `amax` in [2^14, 2^15) (1 for zero or non-finite amax). The GEMMs scale
// dequantized values by `up` = 2^f and outputs by `down` = 2^-f.
struct F16Range {
  const float* row = nullptr;  // activation row factors 2^-e_r (launch_activations_f16)
  float up = 1.0f, down = 1.0f;
};
void weight_f16_factors(float amax, float* up, float* down);

// out[0] = max |x[i]| over n floats (n % 4 == 0) as f32 bits (NaN ignored); out[0] must
// hold 0 (or an earlier maximum) before the launch.
void launch_absmax(const float* x, uint64_t n, uint32_t* out, hipStream_t stream);

// Split-K across work-groups for the LDS-staged GEMV: ks work-groups share
// each 64-row block; partials holds ks * m * 2 * (row blocks * 64) f32 and
// counters one zero-initialised u32 per row block (each launch leaves them
// zero again). ks == 1 needs neither. narrow: 1 = the 16-row form instead
// (no K split; used when its LDS fits), 0 = never, -1 = where the 64-row
// form would split K.
struct GemvSplitK {
  float* partials = nullptr;
  uint32_t* counters = nullptr;
  int ks = 1;
  int narrow = -1;
};
int gemv_default_ksplit(uint64_t rows, uint64_t nb);

// The matmul kernels write y[i][n] = product [+ addend[i * addend_stride + n]]
// (addend may be null; stride 0 broadcasts one row, as a bias).

// The launch the pre-quantized int8 decode GEMV takes: its form, waves per
// work-group (clamped to the form's launch bound), grid and dynamic LDS.
constexpr int kGemvFormLanes8 = 1;  // variant 1: 8 lanes per row
constexpr int kGemvFormRows = 2;    // variant 2: one row per lane, scalar activations
constexpr int kGemvFormLds = 3;     // variant 3: 64 rows per work-group, activations in LDS, split-K
constexpr int kGemvFormNarrow = 4;  // variant 3's 16-row form (long rows, few output rows)
constexpr int kGemvFormWave = 5;    // variant 3 with one super-block per wave (no K split)
struct GemvShape {
  int form = 0;
  int waves = 0;
  unsigned grid_x = 0, grid_y = 1;
  size_t lds = 0;
};
GemvShape gemv_int8_shape(int type, uint64_t rows, uint64_t nb, uint64_t m, int splits, int variant,
                          const GemvSplitK& sk);

// Decode GEMV, m in 1..8, int8 activations. variant 1: 8 lanes per row
// (any m); variant 2: one row per lane, activations through scalar loads
// (m <= 4); 3: row per lane with the activations staged in LDS (m <= 8,
// split-K per `sk`); 0: choose. `splits` = waves per work-group (< 1: choose).
void launch_gemv_int8(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb,
                      const int8_t* values, const float* scales, const int32_t* sums,
                      uint64_t m, float* y, const float* addend, uint64_t addend_stride, int splits,
                      int variant, const GemvSplitK& sk, hipStream_t stream);

// Decode GEMV with the int8 quantization fused in (m <= 8, LDS need <= 64 KiB):
// the work-group quantizes x into LDS and multiplies, one launch. Returns
// false (nothing launched) when the shape does not fit.
bool launch_gemv_fused(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, const float* x,
                       uint64_t m, float* y, const float* addend, uint64_t addend_stride, int splits,
                       const GemvSplitK& sk, hipStream_t stream);

// Decode-step fusions of the fused-quantization GEMV (m = 1; Q4_K and
// IQ4_XS). norm: rmsnorm the activation row with norm_w, norm_eps before
// quantizing it. epilogue 1 (rope): rows below rope_rows rotated in
// interleaved pairs of heads of rope_dim at `position` with frequencies
// freq[rope_dim / 2], and row r written to seg_out[i][r - seg_begin[i]] for
// the segment i holding it (seg_begin[0] = 0, y unused); epilogue 2 (silu
// pairs): stored rows interleave gate / up in blocks of 32 (rows % 64 == 0)
// and y[j] = silu(gate_j) * up_j. Returns false (nothing launched) when the
// shape does not fit the LDS form.
struct GemvFusion {
  const float* norm_w = nullptr;
  float norm_eps = 0.0f;
  const float* freq = nullptr;
  float position = 0.0f;
  uint32_t rope_rows = 0, rope_dim = 2;
  uint32_t seg_begin[3] = {0, 0, 0};
  float* seg_out[3] = {nullptr, nullptr, nullptr};
};
bool launch_gemv_decode_fused(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, const float* x, float* y,
                              bool norm, int epilogue, const GemvFusion& fusion, const GemvSplitK& sk,
                              hipStream_t stream);

// Decode GEMV, m in 1..8, f32 activations.
void launch_gemv_f32(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb,
                     const float* x, uint64_t m, float* y, const float* addend, uint64_t addend_stride,
                     int splits, hipStream_t stream);

// Prefill GEMM on MFMA: y[m][rows] = a16[m][K] . dequant(W)^T, f32 out.
// variant 1: B dequantized through LDS (128 x 128 tiles); 2, 3, 4: B in
// registers with 128 x 256, 128 x 128 and 64 x 256 tiles; 5 (Q4_K): the
// K-split form, 128 x 256 tiles of 8 waves; 0: choose.
// k = the logical row length; plane formats whose rows end inside a group
// take variant 1. The IQ2 / IQ3 grid formats (raw blocks, the grid tables
// in the device copy) take the register-B form: 128 x 256 tiles for
// variant 2, else 128 x 128.
// part: gemm_splits(...) * m * rows floats of workspace for the split-K
// partials of an under-filled register-B or grid-format GEMM (nullptr: no
// split).
// rg: the activation row factors and the weight's factors; the product is
// (a16 . (up dequant(W))^T) row[r] down, exact powers of two.
void launch_gemm(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, uint64_t k,
                 const uint16_t* a16, uint64_t m, float* y, const float* addend, uint64_t addend_stride,
                 int variant, hipStream_t stream, F16Range rg, float* part = nullptr);
// Split-K factor of that GEMM (register-B and grid-format forms; 1: none).
int gemm_splits(int type, uint64_t rows, uint64_t m, uint64_t nb, uint64_t k, int variant);
int gemm_default_variant(int type, uint64_t rows, uint64_t m, uint64_t nb);

// IQ2 / IQ3 grid formats (raw checkpoint blocks; mq_device.h). The grid
// tables (kGridTableBytes, layout in mq_device.h) are copied to this
// device's copy, synchronously on `stream`.
hipError_t grid_tables_upload(const uint8_t* host, hipStream_t stream);
void launch_dequantize_grid(int type, const uint8_t* w, uint64_t rows, uint64_t nb, int logical, float* out,
                            hipStream_t stream);
// m <= 8 rows; int8: xv [m][k] int8 + xs [m][k / 32] scales (quantized
// activations), else xf [m][k] f32.
void launch_gemv_grid(int type, const uint8_t* w, uint64_t nb, uint64_t rows, const int8_t* xv, const float* xs,
                      const float* xf, uint64_t m, int int8, float* y, const float* addend, uint64_t addend_stride,
                      hipStream_t stream);

// Plane formats (Q8_0, Q4_0, IQ4_NL, Q5_K, Q6_K; layout in mq_device.h).
// k is the logical row length (a multiple of the format's block), nb =
// ceil(k / 256) groups.
void launch_repack_planes(int type, const uint8_t* raw, uint64_t rows, uint64_t k, uint64_t nb,
                          uint8_t* tiled, hipStream_t stream);
void launch_dequantize_planes(int type, const uint8_t* tiled, uint64_t rows, uint64_t k, uint64_t nb,
                              int logical, float* out, hipStream_t stream);
// The fewest K-splits whose LDS staging fits 64 KiB for m rows.
int gemv_planes_min_ksplit(uint64_t nb, uint64_t m);
// Decode GEMV (m in 1..8), int8 activations: quantized in the kernel from x
// (x != null) or taken pre-quantized (values, scales, sums).
void launch_gemv_planes_int8(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, uint64_t k,
                             const int8_t* values, const float* scales, const int32_t* sums, const float* x,
                             uint64_t m, float* y, const float* addend, uint64_t addend_stride, int splits,
                             const GemvSplitK& sk, hipStream_t stream);
// Decode GEMV (m in 1..8), f32 activations.
void launch_gemv_planes_f32(int type, const uint8_t* tiled, uint64_t rows, uint64_t nb, uint64_t k,
                            const float* x, uint64_t m, float* y, const float* addend, uint64_t addend_stride,
                            int splits, hipStream_t stream);

// Embedding lookup of `count` token ids (validated, on the device) in a
// packed table of any format: stored rows are the tokens (transposed == 0,
// out[t] = row ids[t]) or the `dim` stored rows hold every token's value
// (transposed != 0). out[count][dim] times `scale` when `scaled`.
void launch_embedding(int type, const uint8_t* tiled, uint64_t nb, int transposed, const uint32_t* ids,
                      uint64_t count, uint64_t dim, float scale, int scaled, float* out, hipStream_t stream);

// Input-major product y[m][n] = x[m][k] . W, W's k stored rows the input
// rows (any format, f32 activations), K-split `ks` ways through `part`
// (ks * 4 * n floats); the splits are added in order [+ addend].
int axpy_ksplit(uint64_t k, uint64_t n);
void launch_axpy(int type, const uint8_t* tiled, uint64_t nb, uint64_t k, uint64_t n, const float* x, uint64_t m,
                 float* y, const float* addend, uint64_t addend_stride, float* part, int ks, hipStream_t stream);

// Grid-shape helper for the GEMV (waves per work-group).
int gemv_default_splits(uint64_t rows, uint64_t nb, uint64_t m, int variant);

}  // namespace mq
