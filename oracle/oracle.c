/*
 * CPU oracle: a plain-C restatement of the reference's packed-weight
 * decode, int8 activation quantizer, scalar column kernel and dense f32
 * matmul. TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Build with -O2 -ffp-contract=off and without -ffast-math: every
 * product and sum below is one IEEE f32 operation, in the reference's
 * order.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* The external `f16_to_f32` (magnetar-provider-api 1.0.0, not vendored;
 * used at src/native/quant.rs:34 and through F16C at quant.rs:1494-1502):
 * IEEE binary16 -> binary32, exact for every pattern. */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t mant = h & 0x3FF;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            /* subnormal: mant * 2^-24, renormalised */
            int e = -1;
            do {
                mant <<= 1;
                e++;
            } while ((mant & 0x400) == 0);
            mant &= 0x3FF;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
        }
    } else if (exp == 31) {
        /* inf, or NaN with its payload kept and the quiet bit set as F16C does */
        bits = sign | 0x7F800000u | (mant << 13) | (mant ? 0x00400000u : 0);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Block geometry (PackedWeightFormat::{block_bytes, block_elements},
 * external; values fixed by the GGUF layouts the decode arms read at
 * quant.rs:102-206: Q8_0 = f16 d + 32 i8; Q4_0 / IQ4_NL = f16 d + 16
 * nibble pairs; Q5_K = d, dmin, 12 scale bytes, 32 high-bit bytes, 128
 * nibble bytes; Q6_K = 128 low, 64 high, 16 i8 scales, f16 d at 208). */
int or_block_bytes(int fmt) {
    switch (fmt) {
    case OR_Q8_0: return 34;
    case OR_Q4_0: return 18;
    case OR_IQ4_NL: return 18;
    case OR_Q2_K: return 84;
    case OR_Q3_K: return 110;
    case OR_Q4_K: return 144;
    case OR_Q5_K: return 176;
    case OR_Q6_K: return 210;
    case OR_IQ4_XS: return 136;
    case OR_IQ2_XXS: return 66;
    case OR_IQ2_XS: return 74;
    case OR_IQ2_S: return 82;
    case OR_IQ3_XXS: return 98;
    case OR_IQ3_S: return 110;
    default: return 0;
    }
}

int or_block_elements(int fmt) {
    switch (fmt) {
    case OR_Q8_0: case OR_Q4_0: case OR_IQ4_NL: return 32;
    case OR_Q2_K: case OR_Q3_K: case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: case OR_IQ4_XS: return 256;
    case OR_IQ2_XXS: case OR_IQ2_XS: case OR_IQ2_S: case OR_IQ3_XXS: case OR_IQ3_S: return 256;
    default: return 0;
    }
}

/* src/native/quant.rs:46-57 (`scale_min_k4`). */
void or_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* The external `iq4_xs_scales` (called at quant.rs:198, 1411): the GGUF
 * IQ4_XS layout, scales_h (u16 LE) then scales_l[4]; run j's 6-bit
 * scale is low nibble j of scales_l plus bits 2j..2j+1 of scales_h, less
 * 32. Parity unpinned by the reference tree (the crate is not vendored). */
void or_iq4_xs_scales(const uint8_t *six, int8_t out[8]) {
    uint32_t h = (uint32_t)six[0] | ((uint32_t)six[1] << 8);
    for (int j = 0; j < 8; j++) {
        int low = (six[2 + j / 2] >> (4 * (j % 2))) & 0xF;
        int high = (h >> (2 * j)) & 3;
        out[j] = (int8_t)((low | (high << 4)) - 32);
    }
}

/* The external `q3_k_scales` (called at quant.rs:167): the GGUF Q3_K
 * packing of sixteen 6-bit scales in 12 bytes, unpacked as ggml does
 * (words a0, a1, t of the bytes: scale i < 4 = low nibble of byte i with
 * bits 2(i % 4)..+1 of t on top, ...). Values 0..63; the caller subtracts
 * 32. Parity unpinned by the reference tree (the crate is not vendored). */
void or_q3_k_scales(const uint8_t *twelve, int8_t out[16]) {
    uint32_t a[3];
    memcpy(a, twelve, 12);
    const uint32_t k1 = 0x03030303u, k2 = 0x0f0f0f0fu, t = a[2];
    uint32_t w[4];
    w[0] = (a[0] & k2) | (((t >> 0) & k1) << 4);
    w[1] = (a[1] & k2) | (((t >> 2) & k1) << 4);
    w[2] = ((a[0] >> 4) & k2) | (((t >> 4) & k1) << 4);
    w[3] = ((a[1] >> 4) & k2) | (((t >> 6) & k1) << 4);
    memcpy(out, w, 16);
}

/* The external `IQ4_NL_VALUES` (quant.rs:185, 201-202): the GGUF
 * kvalues_iq4nl codebook. Parity unpinned by the reference tree. */
static const int8_t IQ4NL[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                 1,    13,   25,  38,  53,  69,  89,  113};

const int8_t *or_iq4nl_values(void) { return IQ4NL; }

/* The external `Q4_0_VALUES` (quant.rs:183, 1626): index i stands for
 * i - 8 ("its quants standing for `q - 8`", quant.rs:180). */
static const int8_t Q40[16] = {-8, -7, -6, -5, -4, -3, -2, -1,
                               0,  1,  2,  3,  4,  5,  6,  7};

const int8_t *or_q4_0_values(void) { return Q40; }

static float half_at(const uint8_t *b, int at) {
    return or_f16_to_f32((uint16_t)(b[at] | (b[at + 1] << 8)));
}

static uint32_t word_at(const uint8_t *b, int at) {
    return (uint32_t)b[at] | ((uint32_t)b[at + 1] << 8) | ((uint32_t)b[at + 2] << 16) | ((uint32_t)b[at + 3] << 24);
}

/* The grid tables, set by the caller (the reference links them from the
 * external crate). */
static uint64_t IQ2XXS_GRID[256], IQ2XS_GRID[512], IQ2S_GRID[1024];
static uint32_t IQ3XXS_GRID[256], IQ3S_GRID[512];

int or_set_iq_grids(const uint64_t *iq2xxs, const uint64_t *iq2xs, const uint64_t *iq2s,
                    const uint32_t *iq3xxs, const uint32_t *iq3s) {
    memcpy(IQ2XXS_GRID, iq2xxs, sizeof IQ2XXS_GRID);
    memcpy(IQ2XS_GRID, iq2xs, sizeof IQ2XS_GRID);
    memcpy(IQ2S_GRID, iq2s, sizeof IQ2S_GRID);
    memcpy(IQ3XXS_GRID, iq3xxs, sizeof IQ3XXS_GRID);
    memcpy(IQ3S_GRID, iq3s, sizeof IQ3S_GRID);
    return 0;
}

/* `iq_signs` (external; the reference tables it at src/native/quant.rs:
 * 986-997 because it is a parity): low 7 bits as given, bit 7 = their
 * parity, so every sign byte negates an even number of values. */
uint8_t or_iq_signs(uint32_t index) {
    uint32_t v = index & 0x7F, p = 0;
    for (int i = 0; i < 7; i++) p ^= (v >> i) & 1;
    return (uint8_t)(v | (p << 7));
}

/* `signed_grid` (src/native/quant.rs:60-69): value j = the grid's byte j as
 * i8, negated where bit j of `signs` is set. */
static void signed_grid(uint64_t grid, uint8_t signs, int8_t *out) {
    for (int j = 0; j < 8; j++) {
        int8_t magnitude = (int8_t)((grid >> (8 * j)) & 0xFF);
        out[j] = ((signs >> j) & 1) ? (int8_t)-magnitude : magnitude;
    }
}

/* `decode` (src/native/quant.rs:96-279): the Q8_0 (102-109), Q4K (110-121),
 * Q5K (122-135), Q6K (136-149), Q2K (150-163), Q3K (164-179), Iq4Nl / Q4_0
 * (180-195), Iq4Xs (196-206) and IQ2 / IQ3 grid (207-277) arms. `run` counts within the block (always 0 for 32-value blocks). */
void or_decode_run(int fmt, const uint8_t *block, int run, int8_t q[OR_RUN],
                   float scale[2], float min[2]) {
    min[0] = min[1] = 0.0f;
    if (fmt == OR_Q8_0) {
        float d = half_at(block, 0);
        for (int i = 0; i < OR_RUN; i++) q[i] = (int8_t)block[2 + i];
        scale[0] = scale[1] = d;
    } else if (fmt == OR_Q4_K || fmt == OR_Q5_K) {
        float d = half_at(block, 0);
        float dmin = half_at(block, 2);
        uint8_t sc, m;
        or_scale_min_k4(run, block + 4, &sc, &m);
        int chunk = run / 2;
        int shift = 4 * (run % 2);
        if (fmt == OR_Q4_K) {
            const uint8_t *qs = block + 16 + 32 * chunk;
            for (int i = 0; i < OR_RUN; i++) q[i] = (int8_t)((qs[i] >> shift) & 0xF);
        } else {
            const uint8_t *low = block + 48 + 32 * chunk;
            const uint8_t *high = block + 16;
            for (int i = 0; i < OR_RUN; i++)
                q[i] = (int8_t)(((low[i] >> shift) & 0xF) | (((high[i] >> run) & 1) << 4));
        }
        float s = d * (float)sc;
        float mn = dmin * (float)m;
        scale[0] = scale[1] = s;
        min[0] = min[1] = mn;
    } else if (fmt == OR_Q6_K) {
        float d = half_at(block, 208);
        int h = run / 4, g = run % 4;
        const uint8_t *low = block + 64 * h + 32 * (g % 2);
        const uint8_t *high = block + 128 + 32 * h;
        int low_shift = 4 * (g / 2), high_shift = 2 * g;
        for (int i = 0; i < OR_RUN; i++)
            q[i] = (int8_t)((int)(((low[i] >> low_shift) & 0xF) | (((high[i] >> high_shift) & 3) << 4)) - 32);
        for (int p = 0; p < 2; p++) scale[p] = d * (float)(int8_t)block[192 + 8 * h + 2 * g + p];
    } else if (fmt == OR_Q2_K) {
        /* quant.rs:150-163 */
        float d = half_at(block, 80), dmin = half_at(block, 82);
        int h = run / 4, j = run % 4;
        const uint8_t *qs = block + 16 + 32 * h;
        for (int i = 0; i < OR_RUN; i++) q[i] = (int8_t)((qs[i] >> (2 * j)) & 3);
        for (int p = 0; p < 2; p++) {
            uint8_t sc = block[8 * h + 2 * j + p];
            scale[p] = d * (float)(sc & 0xF);
            min[p] = dmin * (float)(sc >> 4);
        }
    } else if (fmt == OR_Q3_K) {
        /* quant.rs:164-179 */
        float d = half_at(block, 108);
        int8_t sc[16];
        or_q3_k_scales(block + 96, sc);
        int h = run / 4, j = run % 4;
        const uint8_t *quants = block + 32 + 32 * h;
        const uint8_t *mask = block;
        int bit = 4 * h + j;
        for (int i = 0; i < OR_RUN; i++)
            q[i] = (int8_t)((int)(((quants[i] >> (2 * j)) & 3) | (((mask[i] >> bit) & 1) << 2)) - 4);
        for (int p = 0; p < 2; p++) scale[p] = d * (float)(sc[8 * h + 2 * j + p] - 32);
    } else if (fmt == OR_IQ4_NL || fmt == OR_Q4_0) {
        const int8_t *table = fmt == OR_Q4_0 ? Q40 : IQ4NL;
        float d = half_at(block, 0);
        for (int l = 0; l < 16; l++) {
            uint8_t byte = block[2 + l];
            q[l] = table[byte & 0xF];
            q[l + 16] = table[byte >> 4];
        }
        scale[0] = scale[1] = d;
    } else if (fmt == OR_IQ2_XXS) {
        /* quant.rs:207-218 */
        float d = half_at(block, 0);
        uint32_t grids = word_at(block, 2 + 8 * run), aux = word_at(block, 6 + 8 * run);
        for (int l = 0; l < 4; l++)
            signed_grid(IQ2XXS_GRID[(grids >> (8 * l)) & 0xFF], or_iq_signs(aux >> (7 * l)), q + 8 * l);
        float s = d * (0.5f + (float)(aux >> 28)) * 0.25f;
        scale[0] = scale[1] = s;
    } else if (fmt == OR_IQ2_XS) {
        /* quant.rs:219-232 */
        float d = half_at(block, 0);
        for (int l = 0; l < 4; l++) {
            int at = 2 + 2 * (4 * run + l);
            uint32_t code = (uint32_t)block[at] | ((uint32_t)block[at + 1] << 8);
            signed_grid(IQ2XS_GRID[code & 511], or_iq_signs(code >> 9), q + 8 * l);
        }
        for (int p = 0; p < 2; p++) {
            uint8_t sc = (block[66 + run] >> (4 * p)) & 0xF;
            scale[p] = d * (0.5f + (float)sc) * 0.25f;
        }
    } else if (fmt == OR_IQ2_S) {
        /* quant.rs:233-250 */
        float d = half_at(block, 0);
        for (int l = 0; l < 4; l++) {
            int index = block[2 + 4 * run + l] | (((block[66 + run] >> (2 * l)) & 3) << 8);
            signed_grid(IQ2S_GRID[index], block[34 + 4 * run + l], q + 8 * l);
        }
        for (int p = 0; p < 2; p++) {
            uint8_t sc = (block[74 + run] >> (4 * p)) & 0xF;
            scale[p] = d * (0.5f + (float)sc) * 0.25f;
        }
    } else if (fmt == OR_IQ3_XXS) {
        /* quant.rs:251-262 */
        float d = half_at(block, 0);
        uint32_t aux = word_at(block, 66 + 4 * run);
        for (int l = 0; l < 4; l++) {
            uint64_t low = IQ3XXS_GRID[block[2 + 8 * run + 2 * l]];
            uint64_t high = IQ3XXS_GRID[block[3 + 8 * run + 2 * l]];
            signed_grid(low | (high << 32), or_iq_signs(aux >> (7 * l)), q + 8 * l);
        }
        float s = d * (0.5f + (float)(aux >> 28)) * 0.5f;
        scale[0] = scale[1] = s;
    } else if (fmt == OR_IQ3_S) {
        /* quant.rs:263-277 */
        float d = half_at(block, 0);
        for (int l = 0; l < 4; l++) {
            int i0 = 2 * l, i1 = 2 * l + 1;
            int index0 = block[2 + 8 * run + i0] | (((block[66 + run] >> i0) & 1) << 8);
            int index1 = block[2 + 8 * run + i1] | (((block[66 + run] >> i1) & 1) << 8);
            uint64_t low = IQ3S_GRID[index0], high = IQ3S_GRID[index1];
            signed_grid(low | (high << 32), block[74 + 4 * run + l], q + 8 * l);
        }
        uint8_t sc = (block[106 + run / 2] >> (4 * (run % 2))) & 0xF;
        float s = d * (float)(1 + 2 * sc);
        scale[0] = scale[1] = s;
    } else {
        float d = half_at(block, 0);
        int8_t ls[8];
        or_iq4_xs_scales(block + 2, ls);
        float s = d * (float)ls[run];
        for (int l = 0; l < 16; l++) {
            uint8_t byte = block[8 + 16 * run + l];
            q[l] = IQ4NL[byte & 0xF];
            q[l + 16] = IQ4NL[byte >> 4];
        }
        scale[0] = scale[1] = s;
    }
}

/* RunReader addressing (quant.rs:284-338) and `dequantize_row`
 * (quant.rs:1702-1711): value = scale[p] * q - min[p], p = i / 16. */
int or_dequantize_rows(int fmt, const uint8_t *bytes, uint64_t rows,
                       uint64_t cols, float *out) {
    int bb = or_block_bytes(fmt), be = or_block_elements(fmt);
    if (!bb || cols % (uint64_t)be) return -1;
    int rpb = be / OR_RUN;
    uint64_t row_bytes = cols / be * (uint64_t)bb;
    int8_t q[OR_RUN];
    float scale[2], min[2];
    for (uint64_t r = 0; r < rows; r++) {
        for (uint64_t u = 0; u < cols / OR_RUN; u++) {
            const uint8_t *block = bytes + r * row_bytes + (u / rpb) * bb;
            or_decode_run(fmt, block, (int)(u % rpb), q, scale, min);
            float *o = out + r * cols + u * OR_RUN;
            for (int i = 0; i < OR_RUN; i++) {
                int p = i / 16;
                float v = scale[p] * (float)q[i];
                o[i] = v - min[p];
            }
        }
    }
    return 0;
}

/* Rust `f32 as i8`: saturating, NaN -> 0. */
static int8_t sat_i8(float v) {
    if (isnan(v)) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

/* `quantize_rows` (quant.rs:350-378): per 32-value block,
 * amax = fold(0, f32::max(|x|)) (f32::max ignores NaN, as fmaxf does),
 * d = amax / 127 (true division), q = round_ties_even(x / d) as i8
 * (0 when amax == 0), sums of each 16-value half. */
void or_quantize_rows(const float *x, uint64_t n, int8_t *values,
                      float *scales, int32_t *sums) {
    for (uint64_t b = 0; b < n / OR_RUN; b++) {
        const float *blk = x + b * OR_RUN;
        float amax = 0.0f;
        for (int i = 0; i < OR_RUN; i++) amax = fmaxf(amax, fabsf(blk[i]));
        float d = amax / 127.0f;
        int32_t s[2] = {0, 0};
        for (int i = 0; i < OR_RUN; i++) {
            int8_t q = 0;
            if (amax != 0.0f) q = sat_i8(nearbyintf(blk[i] / d));
            values[b * OR_RUN + i] = q;
            s[i / 16] += q;
        }
        scales[b] = d;
        sums[2 * b] = s[0];
        sums[2 * b + 1] = s[1];
    }
}

/* `int8_rounded` (src/native/tests.rs:77-89): the activations as int8
 * activations see them, f32::from(q) * d. */
void or_int8_rounded(const float *x, uint64_t n, float *out) {
    for (uint64_t b = 0; b < n / OR_RUN; b++) {
        int8_t v[OR_RUN];
        float d;
        int32_t s[2];
        or_quantize_rows(x + b * OR_RUN, OR_RUN, v, &d, s);
        for (int i = 0; i < OR_RUN; i++) out[b * OR_RUN + i] = (float)v[i] * d;
    }
}

/* `dot_halves_scalar` (quant.rs:380-388). */
void or_dot_halves(const int8_t *q, const int8_t *a, int32_t out[2]) {
    out[0] = out[1] = 0;
    for (int i = 0; i < OR_RUN; i++) out[i / 16] += (int32_t)q[i] * (int32_t)a[i];
}

/* The scalar int8 / f32 column loop of `columns::<F>`
 * (quant.rs:559-597). */
int or_columns_scalar(int fmt, const uint8_t *bytes, uint64_t n, uint64_t k,
                      const float *x, uint64_t m, int int8,
                      uint64_t first, uint64_t count, float *out) {
    int bb = or_block_bytes(fmt), be = or_block_elements(fmt);
    if (!bb || k % (uint64_t)be || first + count > n) return -1;
    int rpb = be / OR_RUN;
    uint64_t runs = k / OR_RUN;
    uint64_t row_bytes = k / be * (uint64_t)bb;
    int8_t *qv = 0;
    float *qs = 0;
    int32_t *qsum = 0;
    if (int8) {
        qv = (int8_t *)malloc(m * k);
        qs = (float *)malloc(m * runs * sizeof(float));
        qsum = (int32_t *)malloc(m * runs * 2 * sizeof(int32_t));
        if (!qv || !qs || !qsum) {
            free(qv); free(qs); free(qsum);
            return -2;
        }
        or_quantize_rows(x, m * k, qv, qs, qsum);
    }
    float *acc = (float *)calloc(m ? m : 1, sizeof(float));
    int8_t q[OR_RUN];
    float scale[2], min[2];
    for (uint64_t c = 0; c < count; c++) {
        for (uint64_t r = 0; r < m; r++) acc[r] = 0.0f;
        for (uint64_t u = 0; u < runs; u++) {
            const uint8_t *block = bytes + (first + c) * row_bytes + (u / rpb) * bb;
            or_decode_run(fmt, block, (int)(u % rpb), q, scale, min);
            for (uint64_t r = 0; r < m; r++) {
                uint64_t blk = r * runs + u;
                if (int8) {
                    int32_t dots[2];
                    or_dot_halves(q, qv + blk * OR_RUN, dots);
                    float d = qs[blk];
                    float t = scale[0] * (float)dots[0];
                    t = t + scale[1] * (float)dots[1];
                    t = t - min[0] * (float)qsum[2 * blk];
                    t = t - min[1] * (float)qsum[2 * blk + 1];
                    acc[r] += d * t;
                } else {
                    const float *xa = x + blk * OR_RUN;
                    for (int i = 0; i < OR_RUN; i++) {
                        int p = i / 16;
                        float w = scale[p] * (float)q[i];
                        w = w - min[p];
                        acc[r] += w * xa[i];
                    }
                }
            }
        }
        for (uint64_t r = 0; r < m; r++) out[r * count + c] = acc[r];
    }
    free(acc);
    free(qv);
    free(qs);
    free(qsum);
    return 0;
}

/* Dense `matmul` (src/lib.rs:262-318): row -> inner -> col, f32, no
 * zero-skip, transposes by stride swap. */
int or_matmul_dense(const float *a, uint64_t a_rows, uint64_t a_cols,
                    const float *b, uint64_t b_rows, uint64_t b_cols,
                    int transpose_a, int transpose_b, float *out) {
    uint64_t m = transpose_a ? a_cols : a_rows;
    uint64_t k = transpose_a ? a_rows : a_cols;
    uint64_t k2 = transpose_b ? b_cols : b_rows;
    uint64_t n = transpose_b ? b_rows : b_cols;
    if (k != k2) return -1;
    uint64_t a_row_stride = transpose_a ? 1 : a_cols;
    uint64_t a_inner_stride = transpose_a ? a_cols : 1;
    uint64_t b_inner_stride = transpose_b ? 1 : b_cols;
    uint64_t b_col_stride = transpose_b ? b_cols : 1;
    memset(out, 0, m * n * sizeof(float));
    for (uint64_t row = 0; row < m; row++) {
        float *o = out + row * n;
        for (uint64_t inner = 0; inner < k; inner++) {
            float av = a[row * a_row_stride + inner * a_inner_stride];
            uint64_t base = inner * b_inner_stride;
            for (uint64_t col = 0; col < n; col++) o[col] += av * b[base + col * b_col_stride];
        }
    }
    return 0;
}
