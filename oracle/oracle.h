/*
 * CPU oracle for the GGUF block-quantized matmul path (Q4_K, IQ4_XS,
 * Q8_0, Q4_0, IQ4_NL, Q2_K, Q3_K, Q5_K, Q6_K).
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: tests, the
 * smoke check and bench.py's CPU-baseline leg load it; the product
 * library never links or calls it.
 *
 * Every function restates the reference's Rust algorithm in plain C and
 * cites the file:line it follows (paths relative to the reference repo
 * root). Compiled with -ffp-contract=off: the reference never contracts a
 * multiply and an add into an FMA unless it calls an explicit fmadd.
 */
#ifndef MAGNETAR_ORACLE_H
#define MAGNETAR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (public GGUF spec) */
#define OR_Q4_0 2
#define OR_Q8_0 8
#define OR_Q2_K 10
#define OR_Q3_K 11
#define OR_Q4_K 12
#define OR_Q5_K 13
#define OR_Q6_K 14
#define OR_IQ4_NL 20
#define OR_IQ4_XS 23
#define OR_IQ2_XXS 16
#define OR_IQ2_XS 17
#define OR_IQ3_XXS 18
#define OR_IQ3_S 21
#define OR_IQ2_S 22

/* Values per run (src/native/quant.rs:18-19). */
#define OR_RUN 32

float or_f16_to_f32(uint16_t bits);
int or_block_bytes(int fmt);
int or_block_elements(int fmt);
void or_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m);
void or_iq4_xs_scales(const uint8_t *six, int8_t out[8]);
const int8_t *or_iq4nl_values(void);
const int8_t *or_q4_0_values(void);
void or_q3_k_scales(const uint8_t *twelve, int8_t out[16]);

/* The IQ2 / IQ3 grid tables (magnetar-provider-api `iq_grids`, external):
 * the decode of those formats reads them from here. Entries: IQ2_XXS 256,
 * IQ2_XS 512, IQ2_S 1024 (u64: 8 magnitudes), IQ3_XXS 256, IQ3_S 512 (u32:
 * 4 magnitudes). Copied; returns 0. */
int or_set_iq_grids(const uint64_t *iq2xxs, const uint64_t *iq2xs, const uint64_t *iq2s,
                    const uint32_t *iq3xxs, const uint32_t *iq3s);
/* `iq_signs` (external): the 7-bit index with its parity in bit 7. */
uint8_t or_iq_signs(uint32_t index);

/* Run `run` of one block: 32 signed values, per-half scale and min. */
void or_decode_run(int fmt, const uint8_t *block, int run, int8_t q[OR_RUN],
                   float scale[2], float min[2]);

/* Stored rows of a packed weight dequantized to f32, stored layout. */
int or_dequantize_rows(int fmt, const uint8_t *bytes, uint64_t rows,
                       uint64_t cols, float *out);

/* Activation int8 quantization per 32-value block. */
void or_quantize_rows(const float *x, uint64_t n, int8_t *values,
                      float *scales, int32_t *sums);
void or_int8_rounded(const float *x, uint64_t n, float *out);
void or_dot_halves(const int8_t *q, const int8_t *a, int32_t out[2]);

/* The scalar column kernel: out[r*count + c] for columns first..first+count
 * of a x W (W stored output-major: n stored rows of k). */
int or_columns_scalar(int fmt, const uint8_t *bytes, uint64_t n, uint64_t k,
                      const float *x, uint64_t m, int int8,
                      uint64_t first, uint64_t count, float *out);

/* The dense f32 matmul oracle; returns 0 or -1 on an inner-size mismatch. */
int or_matmul_dense(const float *a, uint64_t a_rows, uint64_t a_cols,
                    const float *b, uint64_t b_rows, uint64_t b_cols,
                    int transpose_a, int transpose_b, float *out);

/* CPU baseline: the reference's default AVX2 path (int8 activations,
 * Q4_K / IQ4_XS specialised column kernels) across a persistent pool of
 * `threads` threads, caller participating. out is m x n. */
int bl_packed_matmul(int fmt, const uint8_t *bytes, uint64_t n, uint64_t k,
                     const float *x, uint64_t m, int threads, float *out);
int bl_has_avx2(void);
float bl_half_f16c(uint16_t bits);

/* Decoder-layer operators (layer.c). Return 0, or -1 on a shape or
 * argument the reference rejects. */
int or_rmsnorm(const float *x, uint64_t rows, uint64_t cols, const float *w, uint64_t w_rows, float epsilon,
               float *out);
int or_rope(const float *x, uint64_t rows, uint64_t cols, float base, float scale, uint64_t dimension,
            uint64_t position_offset, uint64_t head_count, int half_split, float *out);
int or_kv_write(float *store, uint64_t capacity, uint64_t width, const float *rows, uint64_t count,
                uint64_t row_offset);
/* scores: kv_seq floats of scratch */
int or_attention(const float *q, uint64_t seq, const float *k, const float *v, uint64_t kv_seq, uint64_t heads,
                 uint64_t head_dim, uint64_t kv_heads, int causal, float score_scale, float *scores,
                 float *out);
void or_silu_mul(const float *gate, const float *up, uint64_t n, float *out);
int or_add(const float *a, uint64_t n, const float *b, uint64_t b_n, float *out);

#ifdef __cplusplus
}
#endif
#endif
