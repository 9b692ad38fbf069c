/*
 * CPU baseline: the reference's default optimized CPU path restated in C
 * with AVX2/FMA/F16C intrinsics, for timing beside the GPU. TEST AND
 * BENCHMARK INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg and tests).
 *
 * Follows:
 *  - `NativeState::packed_matmul` (src/native/mod.rs:110-152): serial int8
 *    quantization on the caller, columns split into
 *    chunk = max(8, ceil(n / (4 T))) column tasks, per-task local output
 *    scattered into the result;
 *  - `Pool` (src/native/pool.rs:58-155): persistent workers, atomic task
 *    claiming, the caller participates, `run` returns after the last task;
 *  - `columns_q4k_avx2` (src/native/quant.rs:666-744) and
 *    `columns_iq4xs_avx2` + `iq4_pair` + `accumulate_signed`
 *    (quant.rs:956-984, 1364-1433), with `hsum` (quant.rs:905-917).
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

int bl_has_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") &&
           __builtin_cpu_supports("f16c");
}

/* ---- persistent pool (pool.rs) ---------------------------------------- */

typedef void (*task_fn)(void *ctx, size_t index);

typedef struct {
    task_fn fn;
    void *ctx;
    size_t tasks;
    atomic_size_t next;
    atomic_size_t pending;
    int refs; /* workers holding this job, guarded by pool.mu */
} job_t;

typedef struct {
    int threads;
    pthread_t *workers;
    pthread_mutex_t mu;
    pthread_cond_t wake;
    pthread_cond_t done;
    pthread_mutex_t running; /* one run at a time */
    unsigned long generation;
    int shutdown;
    job_t *job;
} pool_t;

static void job_work(pool_t *pool, job_t *job) {
    for (;;) {
        size_t index = atomic_fetch_add(&job->next, 1);
        if (index >= job->tasks) return;
        job->fn(job->ctx, index);
        if (atomic_fetch_sub(&job->pending, 1) == 1) {
            pthread_mutex_lock(&pool->mu);
            pthread_cond_broadcast(&pool->done);
            pthread_mutex_unlock(&pool->mu);
        }
    }
}

static void *worker_main(void *arg) {
    pool_t *pool = (pool_t *)arg;
    unsigned long seen = 0;
    for (;;) {
        pthread_mutex_lock(&pool->mu);
        while (!pool->shutdown && pool->generation == seen)
            pthread_cond_wait(&pool->wake, &pool->mu);
        if (pool->shutdown) {
            pthread_mutex_unlock(&pool->mu);
            return NULL;
        }
        seen = pool->generation;
        job_t *job = pool->job;
        if (job) job->refs++;
        pthread_mutex_unlock(&pool->mu);
        if (job) {
            job_work(pool, job);
            pthread_mutex_lock(&pool->mu);
            job->refs--;
            pthread_cond_broadcast(&pool->done);
            pthread_mutex_unlock(&pool->mu);
        }
    }
}

static pool_t *pool_new(int threads) {
    pool_t *pool = (pool_t *)calloc(1, sizeof(pool_t));
    pool->threads = threads < 1 ? 1 : threads;
    pthread_mutex_init(&pool->mu, NULL);
    pthread_mutex_init(&pool->running, NULL);
    pthread_cond_init(&pool->wake, NULL);
    pthread_cond_init(&pool->done, NULL);
    pool->workers = (pthread_t *)calloc((size_t)pool->threads, sizeof(pthread_t));
    for (int i = 1; i < pool->threads; i++)
        pthread_create(&pool->workers[i], NULL, worker_main, pool);
    return pool;
}

static void pool_run(pool_t *pool, size_t tasks, task_fn fn, void *ctx) {
    if (tasks == 0) return;
    if (tasks == 1 || pool->threads == 1) {
        for (size_t i = 0; i < tasks; i++) fn(ctx, i);
        return;
    }
    pthread_mutex_lock(&pool->running);
    job_t job;
    job.fn = fn;
    job.ctx = ctx;
    job.tasks = tasks;
    atomic_init(&job.next, 0);
    atomic_init(&job.pending, tasks);
    job.refs = 0;
    pthread_mutex_lock(&pool->mu);
    pool->job = &job;
    pool->generation++;
    pthread_cond_broadcast(&pool->wake);
    pthread_mutex_unlock(&pool->mu);
    job_work(pool, &job);
    pthread_mutex_lock(&pool->mu);
    while (atomic_load(&job.pending) != 0 || job.refs != 0)
        pthread_cond_wait(&pool->done, &pool->mu);
    pool->job = NULL;
    pthread_mutex_unlock(&pool->mu);
    pthread_mutex_unlock(&pool->running);
}

/* One pool per thread count, kept for the process (the Provider keeps its
 * pool for its lifetime, mod.rs:525-544). */
static pool_t *cached_pool(int threads) {
    static pthread_mutex_t mu = PTHREAD_MUTEX_INITIALIZER;
    static pool_t *pools[257];
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_mutex_lock(&mu);
    if (!pools[threads]) pools[threads] = pool_new(threads);
    pool_t *p = pools[threads];
    pthread_mutex_unlock(&mu);
    return p;
}

/* ---- AVX2 column kernels ---------------------------------------------- */

__attribute__((target("avx2,fma,f16c"))) static inline float half_f16c(const uint8_t *b) {
    int bits = (int)((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    return _mm_cvtss_f32(_mm_cvtph_ps(_mm_cvtsi32_si128(bits)));
}

/* F16C conversion of one f16 pattern (`half_f16c`, quant.rs:1494-1502),
 * exported to pin the oracle's exact conversion. */
float bl_half_f16c(uint16_t bits) {
    uint8_t b[2] = {(uint8_t)(bits & 0xFF), (uint8_t)(bits >> 8)};
    return half_f16c(b);
}

/* hsum (quant.rs:905-917): (l0+l4, l1+l5, l2+l6, l3+l7), then the high pair
 * onto the low pair, then lane 1 onto lane 0. */
__attribute__((target("avx2,fma,f16c"))) static inline float hsum8(__m256 lanes) {
    __m128 h = _mm_add_ps(_mm256_castps256_ps128(lanes), _mm256_extractf128_ps(lanes, 1));
    h = _mm_add_ps(h, _mm_movehl_ps(h, h));
    return _mm_cvtss_f32(_mm_add_ss(h, _mm_shuffle_ps(h, h, 0x01)));
}

typedef struct {
    const int8_t *values;
    const float *scales;
    const int32_t *sums;
} qrows_t;

/* columns_q4k_avx2 (quant.rs:666-744). */
__attribute__((target("avx2,fma,f16c"))) static void columns_q4k(
    const uint8_t *bytes, size_t row_bytes, const qrows_t *qr, size_t m, size_t k,
    size_t first, size_t count, float *out, __m256 *acc, float *mins) {
    const size_t runs = k / 32, blocks = k / 256;
    const __m256i low_mask = _mm256_set1_epi8(0xF);
    const __m256i ones = _mm256_set1_epi16(1);
    for (size_t c = 0; c < count; c++) {
        for (size_t r = 0; r < m; r++) {
            acc[r] = _mm256_setzero_ps();
            mins[r] = 0.0f;
        }
        const uint8_t *row = bytes + (first + c) * row_bytes;
        for (size_t b = 0; b < blocks; b++) {
            const uint8_t *block = row + b * 144;
            float d = half_f16c(block), dmin = half_f16c(block + 2);
            float scale[8], min[8];
            for (int j = 0; j < 8; j++) {
                uint8_t sc, mn;
                or_scale_min_k4(j, block + 4, &sc, &mn);
                scale[j] = d * (float)sc;
                min[j] = dmin * (float)mn;
            }
            for (int chunk = 0; chunk < 4; chunk++) {
                __m256i raw = _mm256_loadu_si256((const __m256i *)(block + 16 + 32 * chunk));
                __m256i nib[2] = {_mm256_and_si256(raw, low_mask),
                                  _mm256_and_si256(_mm256_srli_epi16(raw, 4), low_mask)};
                for (int half = 0; half < 2; half++) {
                    int j = 2 * chunk + half;
                    size_t u = b * 8 + (size_t)j;
                    for (size_t r = 0; r < m; r++) {
                        size_t index = r * runs + u;
                        __m256i x = _mm256_loadu_si256((const __m256i *)(qr->values + index * 32));
                        __m256 sums = _mm256_cvtepi32_ps(
                            _mm256_madd_epi16(_mm256_maddubs_epi16(nib[half], x), ones));
                        float da = qr->scales[index];
                        acc[r] = _mm256_fmadd_ps(sums, _mm256_set1_ps(da * scale[j]), acc[r]);
                        float t = da * min[j];
                        mins[r] += t * (float)(qr->sums[2 * index] + qr->sums[2 * index + 1]);
                    }
                }
            }
        }
        for (size_t r = 0; r < m; r++) out[r * count + c] = hsum8(acc[r]) - mins[r];
    }
}

/* columns_iq4xs_avx2 (quant.rs:1386-1433) with iq4_pair (1364-1384) and
 * accumulate_signed (956-984). */
__attribute__((target("avx2,fma,f16c"))) static void columns_iq4xs(
    const uint8_t *bytes, size_t row_bytes, const qrows_t *qr, size_t m, size_t k,
    size_t first, size_t count, float *out, __m256 *acc) {
    const size_t runs = k / 32, blocks = k / 256;
    const __m256i mask = _mm256_set1_epi8(0xF);
    const __m256i ones = _mm256_set1_epi16(1);
    const __m128i t128 = _mm_loadu_si128((const __m128i *)or_iq4nl_values());
    const __m256i table = _mm256_set_m128i(t128, t128);
    for (size_t c = 0; c < count; c++) {
        for (size_t r = 0; r < m; r++) acc[r] = _mm256_setzero_ps();
        const uint8_t *row = bytes + (first + c) * row_bytes;
        for (size_t b = 0; b < blocks; b++) {
            const uint8_t *block = row + b * 136;
            float d = half_f16c(block);
            int8_t ls[8];
            or_iq4_xs_scales(block + 2, ls);
            for (int pair = 0; pair < 4; pair++) {
                __m256i raw = _mm256_loadu_si256((const __m256i *)(block + 8 + 32 * pair));
                __m256i lo = _mm256_and_si256(raw, mask);
                __m256i hi = _mm256_and_si256(_mm256_srli_epi16(raw, 4), mask);
                __m256i w[2] = {
                    _mm256_shuffle_epi8(table, _mm256_permute2x128_si256(lo, hi, 0x20)),
                    _mm256_shuffle_epi8(table, _mm256_permute2x128_si256(lo, hi, 0x31))};
                for (int i = 0; i < 2; i++) {
                    int j = 2 * pair + i;
                    float scale = d * (float)ls[j];
                    size_t u = b * 8 + (size_t)j;
                    __m256i mag = _mm256_sign_epi8(w[i], w[i]);
                    for (size_t r = 0; r < m; r++) {
                        size_t index = r * runs + u;
                        __m256i x = _mm256_loadu_si256((const __m256i *)(qr->values + index * 32));
                        __m256 sums = _mm256_cvtepi32_ps(_mm256_madd_epi16(
                            _mm256_maddubs_epi16(mag, _mm256_sign_epi8(x, w[i])), ones));
                        float da = qr->scales[index];
                        acc[r] = _mm256_fmadd_ps(sums, _mm256_set1_ps(da * scale), acc[r]);
                    }
                }
            }
        }
        for (size_t r = 0; r < m; r++) out[r * count + c] = hsum8(acc[r]);
    }
}

/* ---- packed_matmul (mod.rs:110-152) ----------------------------------- */

typedef struct {
    int fmt;
    const uint8_t *bytes;
    size_t row_bytes, n, k, m, chunk;
    qrows_t qr;
    float *out;
} matmul_ctx_t;

static void matmul_task(void *arg, size_t task) {
    matmul_ctx_t *ctx = (matmul_ctx_t *)arg;
    size_t first = task * ctx->chunk;
    size_t count = ctx->n - first < ctx->chunk ? ctx->n - first : ctx->chunk;
    float *local = (float *)malloc(ctx->m * count * sizeof(float));
    __m256 *acc = (__m256 *)aligned_alloc(32, (ctx->m ? ctx->m : 1) * sizeof(__m256));
    float *mins = (float *)malloc((ctx->m ? ctx->m : 1) * sizeof(float));
    if (ctx->fmt == OR_Q4_K)
        columns_q4k(ctx->bytes, ctx->row_bytes, &ctx->qr, ctx->m, ctx->k, first, count, local, acc, mins);
    else
        columns_iq4xs(ctx->bytes, ctx->row_bytes, &ctx->qr, ctx->m, ctx->k, first, count, local, acc);
    for (size_t r = 0; r < ctx->m; r++)
        for (size_t c = 0; c < count; c++) ctx->out[r * ctx->n + first + c] = local[r * count + c];
    free(local);
    free(acc);
    free(mins);
}

int bl_packed_matmul(int fmt, const uint8_t *bytes, uint64_t n, uint64_t k,
                     const float *x, uint64_t m, int threads, float *out) {
    if (!bl_has_avx2()) return -3;
    if ((fmt != OR_Q4_K && fmt != OR_IQ4_XS) || k % 256) return -1;
    pool_t *pool = cached_pool(threads);
    matmul_ctx_t ctx;
    ctx.fmt = fmt;
    ctx.bytes = bytes;
    ctx.row_bytes = k / 256 * (size_t)or_block_bytes(fmt);
    ctx.n = n;
    ctx.k = k;
    ctx.m = m;
    int8_t *values = (int8_t *)malloc(m * k);
    float *scales = (float *)malloc(m * k / 32 * sizeof(float));
    int32_t *sums = (int32_t *)malloc(m * k / 32 * 2 * sizeof(int32_t));
    if (!values || !scales || !sums) {
        free(values); free(scales); free(sums);
        return -2;
    }
    or_quantize_rows(x, m * k, values, scales, sums);
    ctx.qr.values = values;
    ctx.qr.scales = scales;
    ctx.qr.sums = sums;
    ctx.out = out;
    size_t t = (size_t)pool->threads;
    size_t chunk = (n + t * 4 - 1) / (t * 4);
    if (chunk < 8) chunk = 8;
    ctx.chunk = chunk;
    pool_run(pool, (n + chunk - 1) / chunk, matmul_task, &ctx);
    free(values);
    free(scales);
    free(sums);
    return 0;
}
