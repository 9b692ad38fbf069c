/*
 * magnetar_gpu: the MI355X (gfx950) packed-weight matmul behind the
 * Provider's `matmul` Kernel, as a C ABI (libmagnetar_gpu.so).
 *
 * Plain pointers and sizes only. Host pointers are borrowed for the call;
 * device pointers (the *_dev entry points) must be device memory of the
 * context's GPU, and work is enqueued on the given HIP stream (a
 * hipStream_t; NULL is HIP's null stream) and is asynchronous. The
 * host-pointer entry points run on the context's own stream and return
 * when their results are in host memory. Every entry point returns an
 * MQ_* status; on failure mq_last_error() holds the reason. Nothing aborts
 * across the ABI.
 *
 * Each declaration names the reference interface it replaces (paths
 * relative to the reference repository root).
 */
#ifndef MAGNETAR_GPU_H
#define MAGNETAR_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (public GGUF specification) of the packed formats with a
 * GPU path (the reference's PackedWeightFormat variants Q4_0, Q8_0, Q2K,
 * Q3K, Q4K, Q5K, Q6K, Iq4Nl, Iq4Xs; src/native/quant.rs:71-86). */
#define MQ_TYPE_Q4_0 2u
#define MQ_TYPE_Q8_0 8u
#define MQ_TYPE_Q2_K 10u
#define MQ_TYPE_Q3_K 11u
#define MQ_TYPE_Q4_K 12u
#define MQ_TYPE_Q5_K 13u
#define MQ_TYPE_Q6_K 14u
#define MQ_TYPE_IQ4_NL 20u
#define MQ_TYPE_IQ4_XS 23u
#define MQ_TYPE_IQ2_XXS 16u
#define MQ_TYPE_IQ2_XS 17u
#define MQ_TYPE_IQ3_XXS 18u
#define MQ_TYPE_IQ3_S 21u
#define MQ_TYPE_IQ2_S 22u

/* Status codes. */
#define MQ_OK 0
#define MQ_ERR_SHAPE 1     /* KernelError::KernelExecutionFailed (shape) */
#define MQ_ERR_DTYPE 2     /* KernelError::KernelDTypeUnsupported */
#define MQ_DECLINED 3      /* PackedWeightWrite::Declined: caller falls back */
#define MQ_ERR_HIP 4       /* a HIP runtime error */
#define MQ_ERR_OOM 5       /* device allocation failed */
#define MQ_ERR_ARGUMENT 6  /* null pointer, unknown handle, bad flag */

/* matmul flags */
#define MQ_INT8_ACTIVATIONS 1u /* MAGNETAR_CPU_INT8_ACTIVATIONS (default on) */
#define MQ_TRANSPOSE_B 2u      /* the Kernel's transpose_b attribute */

typedef struct mq_ctx mq_ctx;

/* A context on HIP device `device`, with its own stream and workspace.
 * Replaces the executor state `NativeState` built by
 * `NativeCpuExecutor::with_settings` (src/native/mod.rs:525-544). */
int mq_create(int device, mq_ctx **out);

/* Frees every device buffer of the context (src/native/mod.rs:476-497,
 * the executor's Drop). */
void mq_destroy(mq_ctx *ctx);

/* The calling thread's last error on `ctx` (ctx NULL: the thread's last
 * mq_create error). Valid until that thread's next call on the context.
 * Mirrors the `reason` text of KernelError (src/native/mod.rs:119-124). */
const char *mq_last_error(mq_ctx *ctx);

/* Fills the context device's copy of the IQ2 / IQ3 grid tables that the
 * grid formats decode with (`iq_grids::IQ2XXS_GRID` 256, `IQ2XS_GRID` 512,
 * `IQ2S_GRID` 1024 u64 entries of 8 magnitude bytes; `IQ3XXS_GRID` 256,
 * `IQ3S_GRID` 512 u32 entries of 4), synchronously; every context on the
 * device shares them. The reference reads these statics from the external
 * magnetar-provider-api crate (src/native/quant.rs:14, 1057-1061): a Rust
 * binding passes them once at start-up. Waits for all work queued on the
 * device first (every context and stream shares the tables). When every
 * table byte is below 128 (true of the GGUF grids), prefill matmuls of the
 * grid formats run on the MFMA GEMM; otherwise as 8-row decode GEMVs, and
 * mq_matmul_f16_dev declines them. */
int mq_set_iq_grids(mq_ctx *ctx, const uint64_t *iq2xxs, const uint64_t *iq2xs, const uint64_t *iq2s,
                    const uint32_t *iq3xxs, const uint32_t *iq3s);

/* Uploads a packed weight: `stored_rows` rows of `stored_cols` values,
 * `len` = stored_rows * stored_cols / block_values * block_bytes checkpoint
 * bytes (Q8_0 32 / 34, Q4_0 and IQ4_NL 32 / 18, Q2_K 256 / 84, Q3_K
 * 256 / 110, Q4_K 256 / 144, Q5_K 256 / 176, Q6_K 256 / 210, IQ4_XS
 * 256 / 136, IQ2_XXS 256 / 66, IQ2_XS 256 / 74, IQ2_S 256 / 82, IQ3_XXS
 * 256 / 98, IQ3_S 256 / 110); stored_cols must be whole
 * blocks. transposed != 0: the stored rows are the logical [k, n] weight's
 * output columns; 0: an untransposed weight or table whose stored rows are
 * its logical rows. Returns MQ_DECLINED for a type without a GPU path
 * (any other type, and the IQ2 / IQ3 grid formats until mq_set_iq_grids
 * has run on the context's device), so the caller keeps the f32 path.
 * Replaces
 * `write_packed_weight_tensor` -> `PackedWeightWrite::{Stored,Declined}`
 * (src/native/mod.rs:638-653) and `PackedWeight::new` (external,
 * magnetar-provider-api; used at src/native/tests.rs:66). */
int mq_weight_upload(mq_ctx *ctx, uint32_t gguf_type, uint64_t stored_rows,
                     uint64_t stored_cols, int transposed, const uint8_t *bytes,
                     size_t len, uint64_t *handle);

/* Releases a weight's device memory. Replaces `forget_packed` /
 * `release_tensor` (src/native/mod.rs:560-562, 655-660). */
int mq_weight_release(mq_ctx *ctx, uint64_t handle);

/* A weight's format, stored shape and device footprint. The logical shape
 * is [stored_cols, stored_rows] when transposed (`resident_shape`,
 * src/native/mod.rs:459-462). */
int mq_weight_info(mq_ctx *ctx, uint64_t handle, uint32_t *gguf_type,
                   uint64_t *stored_rows, uint64_t *stored_cols, int *transposed,
                   uint64_t *device_bytes);

/* y[m][n] = x[m][k] . W, host pointers, synchronous (returns after y is
 * copied back). The orientation follows the reference's rule
 * (src/native/mod.rs:217-227): when `transposed` (upload) differs from
 * flags & MQ_TRANSPOSE_B the stored rows are the n output columns and k
 * must equal stored_cols (`NativeState::packed_matmul`, mod.rs:110-152 with
 * `quant::matmul_columns`, quant.rs:430-446; flags & MQ_INT8_ACTIVATIONS
 * selects int8 activations, the reference default, else f32); otherwise
 * the stored rows are the k input rows, n = stored_cols, and the product
 * is the input-major one with f32 activations (`packed_axpy`, mod.rs:154-194
 * with `quant::axpy_columns`, quant.rs:1652-1688). A k mismatch is
 * MQ_ERR_SHAPE with the reference's text. */
int mq_matmul(mq_ctx *ctx, uint64_t handle, const float *x, uint64_t m,
              uint64_t k, uint32_t flags, float *y);

/* mq_matmul on device pointers, enqueued on `stream` (a hipStream_t). */
int mq_matmul_dev(mq_ctx *ctx, uint64_t handle, const float *x_dev, uint64_t m,
                  uint64_t k, uint32_t flags, float *y_dev, void *stream);

/* mq_matmul_dev without any device allocation, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). No counterpart in the reference. Every
 * temporary (int8 or f16 activations, split-K partials and counters) lives
 * in one fixed 32 MiB device array per GPU (its address resolved by
 * mq_create), which calls no hipMalloc, hipFree or allocating library
 * routine; a matmul whose temporaries exceed 32 MiB less 64 KiB of
 * counters (e.g. a prefill of m * k * 2 bytes of f16 activations above
 * that) is MQ_ERR_SHAPE. The array is shared by every call on the GPU and
 * keeps the last call's contents (what must start at zero is cleared by
 * each call): calls that overlap on one GPU, on any stream or context,
 * race. Same results as mq_matmul_dev. */
int mq_matmul_noalloc_dev(mq_ctx *ctx, uint64_t handle, const float *x_dev, uint64_t m,
                          uint64_t k, uint32_t flags, float *y_dev, void *stream);

/* y = x . W^T + addend, the addition fused into the kernel's output write
 * (the product rounded first, then the addend added): addend_rows = 1
 * broadcasts one [stored_rows] row (a bias), addend_rows = m adds an
 * [m][stored_rows] tensor (a residual). Replaces the `matmul-bias` /
 * `matmul-residual` epilogue `add` / `residual_add` after `packed_matmul`
 * (src/native/mod.rs:228-235; src/lib.rs:1028-1073, 1128-1133).
 * Host pointers, synchronous. */
int mq_matmul_add(mq_ctx *ctx, uint64_t handle, const float *x, uint64_t m,
                  uint64_t k, uint32_t flags, const float *addend,
                  uint64_t addend_rows, float *y);

/* mq_matmul_add on device pointers, enqueued on `stream`. */
int mq_matmul_add_dev(mq_ctx *ctx, uint64_t handle, const float *x_dev, uint64_t m,
                      uint64_t k, uint32_t flags, const float *addend_dev,
                      uint64_t addend_rows, float *y_dev, void *stream);

/* Int8 activation quantization on device: values[m*k], scales[m*k/32],
 * sums[m*k/32][2] (int32 half sums). Replaces `quant::quantize_rows`
 * (src/native/quant.rs:350-378). */
int mq_quantize_activations_dev(mq_ctx *ctx, const float *x_dev, uint64_t m,
                                uint64_t k, int8_t *values_dev,
                                float *scales_dev, int32_t *sums_dev,
                                void *stream);

/* The decode GEMV on already-quantized activations (m <= 8): the column
 * kernels' int8 path `columns_q4k_avx2` / `columns_iq4xs_avx2`
 * (src/native/quant.rs:666-744, 1386-1433) without the quantization step,
 * so one quantized activation can feed several weights. The stored rows
 * are the outputs, whatever the weight's `transposed`. */
int mq_matmul_prequantized_dev(mq_ctx *ctx, uint64_t handle,
                               const int8_t *values_dev, const float *scales_dev,
                               const int32_t *sums_dev, uint64_t m, uint64_t k,
                               float *y_dev, void *stream);

/* The prefill path's activation operand on device: a16_dev holds m*k f16
 * values, then m f32 row factors (m*k*2 + m*4 bytes; the factors start at
 * the float after the last f16 value). Value (r, c) is f16(v * 2^e_r), v =
 * int8_rounded(x) with MQ_INT8_ACTIVATIONS (the values the reference's
 * int8 activations stand for, `int8_rounded`, src/native/tests.rs:77-89),
 * else x; 2^e_r puts row r's largest magnitude in [2^14, 2^15) (f16's
 * range: up to 65504, full precision from 2^-14), and the row factor is
 * 2^-e_r, which the GEMM applies to its f32 output. */
int mq_prepare_activations_f16_dev(mq_ctx *ctx, const float *x_dev, uint64_t m,
                                   uint64_t k, uint32_t flags, uint16_t *a16_dev,
                                   void *stream);

/* The prefill GEMM on prepared f16 activations (any m, the buffer of
 * mq_prepare_activations_f16_dev): y[m][stored_rows]
 * = a16 . dequantize(W)^T with f32 accumulation, the MFMA replacement of
 * the column kernels for many activation rows
 * (src/native/quant.rs:666-744, 1386-1433 via src/native/mod.rs:110-152).
 * MQ_DECLINED for an IQ2 / IQ3 grid weight whose device grid tables hold a
 * byte of 128 or more (mq_set_iq_grids). */
int mq_matmul_f16_dev(mq_ctx *ctx, uint64_t handle, const uint16_t *a16_dev,
                      uint64_t m, uint64_t k, float *y_dev, void *stream);

/* Bit-exact dequantization into host memory, stored layout
 * [stored_rows][stored_cols] (logical == 0) or the logical transposed
 * layout [stored_cols][stored_rows] (logical != 0). Replaces
 * `PackedWeight::dequantize_stored` / `dequantize` (external) and
 * `quant::dequantize_row` (src/native/quant.rs:1702-1711), reached through
 * `read_tensor` -> `materialize` (src/lib.rs:1615-1620,
 * src/native/mod.rs:196-204). */
int mq_dequantize(mq_ctx *ctx, uint64_t handle, int logical, float *out);

/* mq_dequantize into device memory, enqueued on `stream`. */
int mq_dequantize_dev(mq_ctx *ctx, uint64_t handle, int logical, float *out_dev,
                      void *stream);

/* The `embedding` Kernel on a packed table (src/native/mod.rs:389-417,
 * 432-449): out[count][dim] = the table's logical rows ids[0..count) (the
 * stored rows when the table was uploaded untransposed, else each token's
 * value in every stored row), times `scale` unless scale is NaN (the
 * Kernel's optional `scale` attribute). ids are f32 token ids in host
 * memory, validated first: a negative, fractional or out-of-vocabulary id
 * is MQ_ERR_SHAPE with the reference's text ("token id X is not below the
 * vocabulary size V"). Host output, synchronous. */
int mq_embedding(mq_ctx *ctx, uint64_t handle, const float *ids, uint64_t count,
                 float scale, float *out);

/* mq_embedding into device memory, enqueued on `stream` (the ids are
 * staged synchronously before the kernel is queued). */
int mq_embedding_dev(mq_ctx *ctx, uint64_t handle, const float *ids, uint64_t count,
                     float scale, float *out_dev, void *stream);

/* ---- Decoder-layer operators ------------------------------------------------
 * Device memory, enqueued on `stream` (a hipStream_t; NULL is the null
 * stream). f32, row-major. Floating-point results follow the reference's
 * operators step by step; reductions add in a fixed tree order, so they
 * differ from the reference's left-to-right sums by rounding only. */

#define MQ_ROPE_INTERLEAVED 0 /* pairs (2i, 2i + 1) */
#define MQ_ROPE_HALF_SPLIT 1  /* pairs (i, i + dimension / 2) */

/* out[r] = x[r] * (1 / sqrt(mean(x[r]^2) + epsilon)) * w, w one row
 * (w_rows 1) or one per row (w_rows == rows). Replaces `rmsnorm`
 * (src/lib.rs:348-402) behind the `rmsnorm` Kernel (src/lib.rs:2679-2726). */
int mq_rmsnorm_dev(mq_ctx *ctx, const float *x_dev, uint64_t rows, uint64_t cols,
                   const float *w_dev, uint64_t w_rows, float epsilon, float *out_dev,
                   void *stream);

/* Rotary embedding of `dimension / 2` pairs in each of head_count blocks of
 * every row, at position (position_offset + row) * scale, frequencies
 * base^(-2i/dimension); columns past `dimension` are copied. out may equal
 * x. Replaces `rope_with_pairing` (src/lib.rs:427-687) behind the `rope`
 * Kernel (src/lib.rs:2728-2817) without frequency scaling or a partial
 * rotary factor. */
int mq_rope_dev(mq_ctx *ctx, const float *x_dev, uint64_t rows, uint64_t cols, float base,
                float scale, uint64_t dimension, uint64_t position_offset,
                uint64_t head_count, int pairing, float *out_dev, void *stream);

/* Writes `count` rows of `width` over rows row_offset.. of a store of
 * `capacity` rows, in place. Replaces `kv_write_in_place`
 * (src/lib.rs:740-768) behind the `kv-write` Kernel (src/lib.rs:2531-2537). */
int mq_kv_write_dev(mq_ctx *ctx, float *store_dev, uint64_t capacity, uint64_t width,
                    const float *rows_dev, uint64_t count, uint64_t row_offset, void *stream);

/* Scaled dot-product attention of `seq` query rows q[seq][heads * head_dim]
 * over the first key_count rows of k and v ([kv_rows][kv_heads * head_dim]),
 * the queries being the last `seq` positions; causal masking; grouped-query
 * heads (heads / kv_heads queries share a kv head); score_scale NaN means
 * 1 / sqrt(head_dim). out is [seq][heads * head_dim]. Replaces
 * `attention_with_value_width` (src/lib.rs:780-990) behind the `attention`
 * Kernel with `key_count` (src/lib.rs:2819-2950). head_dim 128 with
 * heads / kv_heads in {1, 2, 4, 8} has a GPU path; other shapes return
 * MQ_DECLINED. */
int mq_attention_dev(mq_ctx *ctx, const float *q_dev, uint64_t seq, const float *k_dev,
                     const float *v_dev, uint64_t kv_rows, uint64_t key_count, uint64_t heads,
                     uint64_t head_dim, uint64_t kv_heads, int causal, float score_scale,
                     float *out_dev, void *stream);

/* out = silu(gate) * up, silu(x) = x * (1 / (1 + exp(-x))). Replaces the
 * `silu-mul` Kernel (src/lib.rs:2592-2596). */
int mq_silu_mul_dev(mq_ctx *ctx, const float *gate_dev, const float *up_dev, uint64_t n,
                    float *out_dev, void *stream);

/* out[i] = a[i] + b[i % b_n], b_n == n or one row broadcast. Replaces `add`
 * / `residual_add` (src/lib.rs:1019-1075, 1128-1133). */
int mq_add_dev(mq_ctx *ctx, const float *a_dev, uint64_t n, const float *b_dev, uint64_t b_n,
               float *out_dev, void *stream);

/* ---- Decode-step fusions ------------------------------------------------------
 * No counterpart in the reference: one launch for a chain of its operators
 * in a one-token decode step, for callers that keep the step on the device.
 * Each part computes what the separate entry points compute (the same
 * operators, rounded the same way; the rmsnorm's sum of squares is added
 * in another tree order). */

#define MQ_EPILOGUE_NONE 0u
#define MQ_EPILOGUE_ROPE_KV 1u    /* rope rows, route rows to Q / K-row / V-row outputs */
#define MQ_EPILOGUE_SILU_PAIRS 2u /* silu(gate) * up of interleaved gate / up rows */

typedef struct {
  /* non-NULL: x is first rmsnorm'd with this [k] weight and norm_epsilon
   * (mq_rmsnorm_dev with w_rows 1) */
  const float *norm_weight;
  float norm_epsilon;
  uint32_t epilogue;
  /* MQ_EPILOGUE_ROPE_KV: output rows [0, rope_rows) are rotated in
   * interleaved pairs, heads of rope_dim, at position rope_offset with
   * rope_base / rope_scale (mq_rope_dev, MQ_ROPE_INTERLEAVED); then rows
   * [seg_begin[i], seg_begin[i + 1]) are written to seg_out[i] (seg_begin[0]
   * = 0, the last segment ends at stored_rows): e.g. Q, the K cache's row,
   * the V cache's row (mq_kv_write_dev). y_dev is unused. */
  uint64_t rope_rows, rope_dim, rope_offset;
  float rope_base, rope_scale;
  uint64_t seg_begin[3];
  float *seg_out[3];
} mq_decode_fusion;

/* One activation row, int8 activations: y = [rmsnorm](x) . W^T with the
 * epilogue. MQ_EPILOGUE_SILU_PAIRS takes a weight whose stored rows
 * interleave gate and up rows in blocks of 32 (block 2i: gate rows 32i..,
 * block 2i + 1: up rows 32i..; stored_rows a multiple of 64) and writes
 * y[j] = silu(gate_j) * up_j, stored_rows / 2 values (mq_silu_mul_dev).
 * Q4_K and IQ4_XS weights; others, or a row too long for the kernel's LDS
 * staging, return MQ_DECLINED. */
int mq_decode_matmul_dev(mq_ctx *ctx, uint64_t handle, const float *x_dev, uint64_t k,
                         const mq_decode_fusion *fusion, float *y_dev, void *stream);

/* ---- Device-resident tensor storage ---------------------------------------------
 * The memory a device Provider keeps its tensors in (placement
 * ProviderOwnedOpaque): the reference stores them in a host map
 * (`ReferenceCpuExecutor::storage`, src/lib.rs:1556-1621); a GPU Provider
 * keeps them in HBM and copies to or from the host only on request
 * (`read_tensor`, `write_tensor`). */

/* The context's own stream (a hipStream_t), the one its host-pointer entry
 * points use; NULL for a NULL context. */
void *mq_context_stream(mq_ctx *ctx);

/* Device memory of the context's GPU (bytes 0: *dev = NULL). */
int mq_device_alloc(mq_ctx *ctx, uint64_t bytes, void **dev);

/* Frees mq_device_alloc memory after the context's stream has drained. */
int mq_device_free(mq_ctx *ctx, void *dev);

/* Host -> device and device -> host copies ordered on the context's stream
 * (after the work queued on it); they return when the copy is done. */
int mq_copy_to_device(mq_ctx *ctx, void *dst_dev, const void *src, uint64_t bytes);
int mq_copy_to_host(mq_ctx *ctx, void *dst, const void *src_dev, uint64_t bytes);

/* Device -> device copy, enqueued on `stream`. */
int mq_copy_dev(mq_ctx *ctx, void *dst_dev, const void *src_dev, uint64_t bytes, void *stream);

/* dst[0..count) = value, a fill kernel enqueued on `stream`. */
int mq_fill_dev(mq_ctx *ctx, float *dst_dev, uint64_t count, float value, void *stream);

/* Waits for the work queued on `stream`. */
int mq_synchronize(mq_ctx *ctx, void *stream);

/* ---- Launch-shape query --------------------------------------------------------
 * No counterpart in the reference (its pool has no launch shape): the launch
 * the pre-quantized int8 decode GEMV (mq_matmul_prequantized_dev) takes for
 * a Q4_K or IQ4_XS weight, computed on the host without a device, for tests
 * and tuning. waves (waves per work-group, < 1: the default), variant (0:
 * the default; 1, 2, 3: the MQ_GEMV_VARIANT forms) and ksplit (< 1: the
 * default K split) are the overrides a context reads from MQ_GEMV_SPLITS,
 * MQ_GEMV_VARIANT and MQ_GEMV_KSPLIT; every form clamps waves to its
 * kernel's launch bound (8 waves, 512 threads; the one-block-per-wave form,
 * taken only without a waves override, 16 waves, 1024 threads). */
#define MQ_GEMV_FORM_LANES8 1u /* 8 lanes per row */
#define MQ_GEMV_FORM_ROWS 2u   /* one row per lane, scalar activation reads (m <= 4) */
#define MQ_GEMV_FORM_LDS 3u    /* 64 rows per work-group, activations in LDS, split-K over grid_y */
#define MQ_GEMV_FORM_NARROW 4u /* 16 rows per work-group, activations in LDS */
#define MQ_GEMV_FORM_WAVE 5u   /* 64 rows per work-group, one super-block per wave (up to 16 waves) */

typedef struct {
  uint32_t form;
  uint32_t waves;  /* work-group = 64 * waves threads */
  uint32_t grid_x, grid_y;
  uint64_t lds_bytes;  /* dynamic LDS per work-group */
} mq_gemv_shape;

int mq_gemv_launch_shape(uint32_t gguf_type, uint64_t stored_rows, uint64_t stored_cols, uint64_t m,
                         int waves, int variant, int ksplit, mq_gemv_shape *out);

/* Library version string. */
const char *mq_version(void);

#ifdef __cplusplus
}
#endif
#endif
