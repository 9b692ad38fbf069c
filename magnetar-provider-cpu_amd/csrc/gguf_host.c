/*
 * Host-side GGUF block encoders and the seeded Gaussian generator.
 *
 * The reference only consumes checkpoint-encoded bytes (its loader
 * builds a PackedWeight from GGUF data, src/native/mod.rs:638-653); it
 * has no quantizer. These encoders produce valid Q4_K / IQ4_XS blocks in
 * the byte layouts the reference decodes (src/native/quant.rs:110-121,
 * 196-206), for benchmarks and tests. Parity never depends on them: the
 * GPU path and the oracle consume the same bytes.
 */
#include "magnetar_gguf.h"

#include <math.h>
#include <string.h>

/* ---- f16 <-> f32 ------------------------------------------------------ */

uint16_t gg_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFF;
    uint32_t mant = x & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u | (mant >> 13) : 0));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant |= 0x800000u;
        int shift = 14 - e; /* 14..24 */
        uint32_t half = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1);
        uint32_t mid = 1u << (shift - 1);
        if (rem > mid || (rem == mid && (half & 1))) half++;
        return (uint16_t)(sign | half);
    }
    uint32_t half = ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1))) half++;
    return (uint16_t)(sign | half);
}

float gg_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1F, mant = h & 0x3FFu, bits;
    if (exp == 0) {
        float v = ldexpf((float)mant, -24);
        return sign ? -v : v;
    }
    if (exp == 31) bits = sign | 0x7F800000u | (mant << 13);
    else bits = sign | ((exp + 112) << 23) | (mant << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* ---- generator --------------------------------------------------------- */

static uint64_t splitmix64(uint64_t *state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void gg_gaussian_f32(uint64_t seed, float sigma, float *out, uint64_t n) {
    uint64_t state = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (uint64_t i = 0; i < n; i += 2) {
        double u1 = ((double)(splitmix64(&state) >> 11) + 0.5) * 0x1.0p-53;
        double u2 = ((double)(splitmix64(&state) >> 11) + 0.5) * 0x1.0p-53;
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(sigma * r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(sigma * r * sin(two_pi * u2));
    }
}

/* ---- geometry ---------------------------------------------------------- */

uint64_t gg_row_bytes(uint32_t gguf_type, uint64_t cols) {
    uint64_t values = 256, bytes = 0;
    switch (gguf_type) {
    case 2: values = 32; bytes = 18; break;   /* Q4_0 */
    case 8: values = 32; bytes = 34; break;   /* Q8_0 */
    case 20: values = 32; bytes = 18; break;  /* IQ4_NL */
    case 10: bytes = 84; break;               /* Q2_K */
    case 11: bytes = 110; break;              /* Q3_K */
    case GG_TYPE_Q4_K: bytes = 144; break;
    case 13: bytes = 176; break;              /* Q5_K */
    case 14: bytes = 210; break;              /* Q6_K */
    case GG_TYPE_IQ4_XS: bytes = 136; break;
    default: return 0;
    }
    return cols % values ? 0 : cols / values * bytes;
}

static int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

/* ---- Q4_K -------------------------------------------------------------- */

/* One 256-weight super-block: per 32-weight sub-block an affine map
 * w ~ s*q - m with q in 0..15, s and m quantized to 6 bits against the
 * block's f16 d and dmin; packed as d | dmin | scales[12] | qs[128]. */
static void encode_q4k_block(const float *w, uint8_t *blk) {
    float scale[8], min[8], max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) {
        float lo = w[32 * j], hi = w[32 * j];
        for (int i = 1; i < 32; i++) {
            if (w[32 * j + i] < lo) lo = w[32 * j + i];
            if (w[32 * j + i] > hi) hi = w[32 * j + i];
        }
        if (lo > 0.0f) lo = 0.0f;
        scale[j] = (hi - lo) / 15.0f;
        min[j] = -lo;
        if (scale[j] > max_scale) max_scale = scale[j];
        if (min[j] > max_min) max_min = min[j];
    }
    uint16_t dh = gg_f32_to_f16(max_scale / 63.0f);
    uint16_t mh = gg_f32_to_f16(max_min / 63.0f);
    float d = gg_f16_to_f32(dh), dmin = gg_f16_to_f32(mh);
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = (uint8_t)(d > 0.0f ? clampi((int)lrintf(scale[j] / d), 0, 63) : 0);
        mn[j] = (uint8_t)(dmin > 0.0f ? clampi((int)lrintf(min[j] / dmin), 0, 63) : 0);
    }
    memset(blk, 0, 144);
    blk[0] = (uint8_t)(dh & 0xFF);
    blk[1] = (uint8_t)(dh >> 8);
    blk[2] = (uint8_t)(mh & 0xFF);
    blk[3] = (uint8_t)(mh >> 8);
    uint8_t *q = blk + 4;
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
    uint8_t *qs = blk + 16;
    for (int j = 0; j < 8; j++) {
        float s = d * (float)sc[j], m = dmin * (float)mn[j];
        for (int i = 0; i < 32; i++) {
            int v = s > 0.0f ? clampi((int)lrintf((w[32 * j + i] + m) / s), 0, 15) : 0;
            qs[32 * (j / 2) + i] |= (uint8_t)(v << (4 * (j % 2)));
        }
    }
}

/* ---- IQ4_XS ------------------------------------------------------------ */

static const int8_t IQ4NL_VALUES[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                        1,    13,   25,  38,  53,  69,  89,  113};

static int nearest_iq4(float v) {
    int best = 0;
    float err = fabsf(v - (float)IQ4NL_VALUES[0]);
    for (int i = 1; i < 16; i++) {
        float e = fabsf(v - (float)IQ4NL_VALUES[i]);
        if (e < err) {
            err = e;
            best = i;
        }
    }
    return best;
}

/* One 256-weight super-block: per 32-weight run a signed scale mapping
 * the run's largest-magnitude weight onto the codebook's -127 end, the
 * scales quantized to 6 bits (ls - 32) against the block's f16 d; packed
 * as d | scales_h (u16) | scales_l[4] | qs[128]. */
static void encode_iq4xs_block(const float *w, uint8_t *blk) {
    float scale[8], big = 0.0f;
    int big_j = 0;
    for (int j = 0; j < 8; j++) {
        float v = 0.0f;
        for (int i = 0; i < 32; i++)
            if (fabsf(w[32 * j + i]) > fabsf(v)) v = w[32 * j + i];
        scale[j] = v / -127.0f;
        if (fabsf(scale[j]) > big) {
            big = fabsf(scale[j]);
            big_j = j;
        }
    }
    uint16_t dh = gg_f32_to_f16(-scale[big_j] / 32.0f);
    float d = gg_f16_to_f32(dh);
    int ls[8];
    for (int j = 0; j < 8; j++) ls[j] = d != 0.0f ? clampi((int)lrintf(scale[j] / d), -32, 31) : 0;
    memset(blk, 0, 136);
    blk[0] = (uint8_t)(dh & 0xFF);
    blk[1] = (uint8_t)(dh >> 8);
    uint32_t high = 0;
    for (int j = 0; j < 8; j++) {
        int u = ls[j] + 32;
        high |= (uint32_t)((u >> 4) & 3) << (2 * j);
        blk[4 + j / 2] |= (uint8_t)((u & 0xF) << (4 * (j % 2)));
    }
    blk[2] = (uint8_t)(high & 0xFF);
    blk[3] = (uint8_t)(high >> 8);
    for (int j = 0; j < 8; j++) {
        float s = d * (float)ls[j];
        for (int l = 0; l < 16; l++) {
            int lo = s != 0.0f ? nearest_iq4(w[32 * j + l] / s) : 8;
            int hi = s != 0.0f ? nearest_iq4(w[32 * j + 16 + l] / s) : 8;
            blk[8 + 16 * j + l] = (uint8_t)(lo | (hi << 4));
        }
    }
}

int gg_quantize(uint32_t gguf_type, const float *w, uint64_t rows, uint64_t cols,
                uint8_t *out) {
    uint64_t row_bytes = gg_row_bytes(gguf_type, cols);
    if (!row_bytes || cols % 256 || (gguf_type != GG_TYPE_Q4_K && gguf_type != GG_TYPE_IQ4_XS)) return -1;
    for (uint64_t r = 0; r < rows; r++) {
        for (uint64_t b = 0; b < cols / 256; b++) {
            const float *src = w + r * cols + b * 256;
            if (gguf_type == GG_TYPE_Q4_K) encode_q4k_block(src, out + r * row_bytes + b * 144);
            else encode_iq4xs_block(src, out + r * row_bytes + b * 136);
        }
    }
    return 0;
}
