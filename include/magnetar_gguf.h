/*
 * Host-side GGUF encoders and seeded synthetic data (libmagnetar_gguf.so).
 *
 * No counterpart in the reference: it only consumes checkpoint-encoded
 * bytes built by the external GGUF loader (src/native/mod.rs:638-653,
 * `write_packed_weight_tensor`). These routines produce such bytes for
 * tests and benchmarks. Host code only: nothing here touches a GPU.
 */
#ifndef MAGNETAR_GGUF_H
#define MAGNETAR_GGUF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids from the public GGUF specification. */
#define GG_TYPE_Q4_K 12u
#define GG_TYPE_IQ4_XS 23u

/* IEEE binary16 <-> binary32 (round to nearest even on the way down). */
uint16_t gg_f32_to_f16(float f);
float gg_f16_to_f32(uint16_t h);

/* n values ~ N(0, sigma^2): splitmix64 (state = seed) feeding Box-Muller in
 * f64, two values per pair of draws, rounded to f32. */
void gg_gaussian_f32(uint64_t seed, float sigma, float *out, uint64_t n);

/* Bytes of one stored row of `cols` weights for Q4_0, Q8_0, IQ4_NL (32-value
 * blocks), Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_XS (256-value blocks); 0 for
 * another type
 * or cols not whole blocks. */
uint64_t gg_row_bytes(uint32_t gguf_type, uint64_t cols);

/* Encodes rows x cols f32 weights (row-major) into gguf_type blocks, rows
 * stored one after another (Q4_K and IQ4_XS only). Returns 0, or -1 for an
 * unsupported type or shape. */
int gg_quantize(uint32_t gguf_type, const float *w, uint64_t rows, uint64_t cols,
                uint8_t *out);

#ifdef __cplusplus
}
#endif
#endif
