/*
 * cpu_baseline.c -- SIMD restatement of rusty_whisper's CPU matmul_t_q
 * (src/quant.rs:754-1051) for timing on the GPU host.  TEST / BENCH
 * INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg and the tests that pin it
 * bitwise to oracle.c's lane emulation); the product never links it.
 *
 * Structure kept from the reference, because the baseline must cost what the
 * reference costs:
 *   - tier chosen at run time: AVX-512 VNNI (avx512vnni+avx512vl) > AVX2 >
 *     f32 dequant fallback (quant.rs:766-770, 995-1018)
 *   - activations quantized serially on every call (quant.rs:766, 691-716)
 *   - a weight's first call takes the cold path (rows re-unpacked per
 *     M-tile into N_BLOCK scratch rows); from the second call on the whole
 *     matrix is int8-unpacked once, in parallel, and cached
 *     (quant.rs:779-786, 589-639)
 *   - N split into hardware_concurrency chunks when m*n*k > 2^20, one thread
 *     per chunk, M_BLOCK=64 / N_BLOCK=8 blocking, x4 row kernels with an x1
 *     remainder, serial copy-back (quant.rs:790-1049, tensor.rs:44-50)
 * Compiled with -ffp-contract=off and per-function target attributes (no
 * -march=native: the GPU host's CPU is not this container's).
 */
#define _GNU_SOURCE
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "oracle.h"

#define QK 32
#define N_BLOCK 8
#define M_BLOCK 64
#define PAR_THRESHOLD (1u << 20)

enum { TIER_VNNI = 0, TIER_AVX2 = 1, TIER_F32 = 2 };

int cb_detect_tier(void)
{
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512vl") &&
        __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"))
        return TIER_VNNI;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"))
        return TIER_AVX2;
    return TIER_F32;
}

/* std::thread::available_parallelism(): the CPUs this process may run on */
int cb_hw_threads(void)
{
    cpu_set_t set;
    if (sched_getaffinity(0, sizeof(set), &set) == 0) {
        int c = CPU_COUNT(&set);
        if (c > 0)
            return c;
    }
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

/* ------------------------------------------------------------ kernels */

#define T_AVX2 __attribute__((target("avx2,fma")))
#define T_VNNI __attribute__((target("avx2,fma,avx512f,avx512vl,avx512vnni")))

T_AVX2 static inline float hsum8(__m256 v)
{
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_hadd_ps(s, s);
    s = _mm_hadd_ps(s, s);
    return _mm_cvtss_f32(s);
}

/* 16 packed bytes -> low nibbles (elements 0..15) and high nibbles (16..31) */
T_AVX2 static inline void split_nibbles(const uint8_t *p, __m128i *lo, __m128i *hi)
{
    __m128i v = _mm_loadu_si128((const __m128i *)p);
    __m128i mask = _mm_set1_epi8(0x0f);
    *lo = _mm_and_si128(v, mask);
    *hi = _mm_and_si128(_mm_srli_epi16(v, 4), mask);
}

/* bits [base, base+16) of qh as 0x10 / 0x00 bytes */
T_AVX2 static inline __m128i qh_flags(uint32_t qh, int base)
{
    uint32_t w = qh >> base;
    __m128i bytes = _mm_set_epi64x((long long)(0x0101010101010101ULL * ((w >> 8) & 0xff)),
                                   (long long)(0x0101010101010101ULL * (w & 0xff)));
    __m128i sel = _mm_set1_epi64x((long long)0x8040201008040201ULL);
    __m128i hit = _mm_cmpeq_epi8(_mm_and_si128(bytes, sel), sel);
    return _mm_and_si128(hit, _mm_set1_epi8(0x10));
}

static inline float f16_at(const uint8_t *p) { return or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }
static inline uint32_t u32_at(const uint8_t *p)
{
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}

/* quant.rs:256-320: one weight row -> int8 quants + per-block d / m */
T_AVX2 static void unpack_row(int dtype, const uint8_t *raw, int bb, size_t nb, int8_t *qb, float *db,
                              float *mb)
{
    for (size_t bl = 0; bl < nb; bl++) {
        const uint8_t *blk = raw + bl * (size_t)bb;
        int8_t *o = qb + bl * QK;
        __m128i lo, hi;
        switch (dtype) {
        case 8:
            _mm256_storeu_si256((__m256i *)o, _mm256_loadu_si256((const __m256i *)(blk + 2)));
            db[bl] = f16_at(blk);
            mb[bl] = 0.0f;
            continue;
        case 2:
            split_nibbles(blk + 2, &lo, &hi);
            lo = _mm_sub_epi8(lo, _mm_set1_epi8(8));
            hi = _mm_sub_epi8(hi, _mm_set1_epi8(8));
            db[bl] = f16_at(blk);
            mb[bl] = 0.0f;
            break;
        case 3:
            split_nibbles(blk + 4, &lo, &hi);
            db[bl] = f16_at(blk);
            mb[bl] = f16_at(blk + 2);
            break;
        case 6: {
            uint32_t qh = u32_at(blk + 2);
            split_nibbles(blk + 6, &lo, &hi);
            lo = _mm_sub_epi8(_mm_or_si128(lo, qh_flags(qh, 0)), _mm_set1_epi8(16));
            hi = _mm_sub_epi8(_mm_or_si128(hi, qh_flags(qh, 16)), _mm_set1_epi8(16));
            db[bl] = f16_at(blk);
            mb[bl] = 0.0f;
            break;
        }
        default: { /* 7 */
            uint32_t qh = u32_at(blk + 4);
            split_nibbles(blk + 8, &lo, &hi);
            lo = _mm_or_si128(lo, qh_flags(qh, 0));
            hi = _mm_or_si128(hi, qh_flags(qh, 16));
            db[bl] = f16_at(blk);
            mb[bl] = f16_at(blk + 2);
            break;
        }
        }
        _mm_storeu_si128((__m128i *)o, lo);
        _mm_storeu_si128((__m128i *)(o + 16), hi);
    }
}

/* quant.rs:403-418 */
T_AVX2 static void block_sums(const int8_t *qb, size_t nb, int32_t *sumb)
{
    __m256i ones = _mm256_set1_epi16(1);
    for (size_t bl = 0; bl < nb; bl++) {
        __m256i b = _mm256_loadu_si256((const __m256i *)(qb + bl * QK));
        __m256i w = _mm256_add_epi32(
            _mm256_madd_epi16(_mm256_cvtepi8_epi16(_mm256_castsi256_si128(b)), ones),
            _mm256_madd_epi16(_mm256_cvtepi8_epi16(_mm256_extracti128_si256(b, 1)), ones));
        __m128i s = _mm_add_epi32(_mm256_castsi256_si128(w), _mm256_extracti128_si256(w, 1));
        s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
        s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
        sumb[bl] = _mm_cvtsi128_si32(s);
    }
}

typedef struct {
    const int8_t *q[4];
    const float *d[4];
    const int32_t *s[4];
} rows4_t;

/* quant.rs:366-395 */
T_AVX2 static void dot_avx2_x4(const rows4_t *a, int nr, const int8_t *qb, const float *db,
                               const float *mb, size_t nb, float *out)
{
    __m256i ones = _mm256_set1_epi16(1);
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(),
                     _mm256_setzero_ps()};
    float corr[4] = {0, 0, 0, 0};
    for (size_t bl = 0; bl < nb; bl++) {
        __m256i b = _mm256_loadu_si256((const __m256i *)(qb + bl * QK));
        __m256i absb = _mm256_sign_epi8(b, b);
        float dbl = db[bl];
        for (int r = 0; r < nr; r++) {
            __m256i x = _mm256_loadu_si256((const __m256i *)(a->q[r] + bl * QK));
            __m256i prod = _mm256_maddubs_epi16(absb, _mm256_sign_epi8(x, b));
            __m256i p32 = _mm256_madd_epi16(prod, ones);
            __m256 scale = _mm256_set1_ps(a->d[r][bl] * dbl);
            acc[r] = _mm256_fmadd_ps(scale, _mm256_cvtepi32_ps(p32), acc[r]);
            corr[r] += mb[bl] * a->d[r][bl] * (float)a->s[r][bl];
        }
    }
    for (int r = 0; r < nr; r++)
        out[r] = hsum8(acc[r]) + corr[r];
}

/* quant.rs:431-490 */
T_VNNI static void dot_vnni_x4(const rows4_t *a, int nr, const int8_t *qb, const float *db,
                               const float *mb, const int32_t *sumb, size_t nb, float *out)
{
    __m256i off = _mm256_set1_epi8((char)0x80);
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(),
                     _mm256_setzero_ps()};
    float corr[4] = {0, 0, 0, 0};
    for (size_t bl = 0; bl < nb; bl++) {
        __m256i b = _mm256_loadu_si256((const __m256i *)(qb + bl * QK));
        float dbl = db[bl], mbl = mb[bl], sbl = (float)sumb[bl];
        for (int r = 0; r < nr; r++) {
            __m256i x = _mm256_loadu_si256((const __m256i *)(a->q[r] + bl * QK));
            __m256i dp = _mm256_dpbusd_epi32(_mm256_setzero_si256(), _mm256_xor_si256(x, off), b);
            float s = a->d[r][bl] * dbl;
            acc[r] = _mm256_fmadd_ps(_mm256_set1_ps(s), _mm256_cvtepi32_ps(dp), acc[r]);
            corr[r] += s * (-128.0f) * sbl + mbl * a->d[r][bl] * (float)a->s[r][bl];
        }
    }
    for (int r = 0; r < nr; r++)
        out[r] = hsum8(acc[r]) + corr[r];
}

/* ----------------------------------------------------------- QTensor */

typedef struct {
    int8_t *q;
    float *d, *m;
    int32_t *sum;
} packed_t;

typedef struct cb_qtensor {
    int dtype, bb;
    size_t n, k, nb;
    uint8_t *raw;
    size_t calls;
    packed_t *packed;
    pthread_mutex_t lock;
} cb_qtensor;

cb_qtensor *cb_qtensor_new(int dtype, size_t n, size_t k, const uint8_t *raw)
{
    int bb = or_block_bytes(dtype);
    if (bb < 0 || k % QK)
        return NULL;
    cb_qtensor *t = (cb_qtensor *)calloc(1, sizeof(*t));
    t->dtype = dtype;
    t->bb = bb;
    t->n = n;
    t->k = k;
    t->nb = k / QK;
    t->raw = (uint8_t *)malloc(n * t->nb * (size_t)bb);
    memcpy(t->raw, raw, n * t->nb * (size_t)bb);
    pthread_mutex_init(&t->lock, NULL);
    return t;
}

void cb_qtensor_free(cb_qtensor *t)
{
    if (!t)
        return;
    if (t->packed) {
        free(t->packed->q);
        free(t->packed->d);
        free(t->packed->m);
        free(t->packed->sum);
        free(t->packed);
    }
    free(t->raw);
    pthread_mutex_destroy(&t->lock);
    free(t);
}

typedef struct {
    const cb_qtensor *t;
    packed_t *p;
    size_t r0, r1;
} pack_job_t;

static void *pack_rows(void *arg)
{
    pack_job_t *j = (pack_job_t *)arg;
    const cb_qtensor *t = j->t;
    for (size_t r = j->r0; r < j->r1; r++) {
        unpack_row(t->dtype, t->raw + r * t->nb * (size_t)t->bb, t->bb, t->nb, j->p->q + r * t->k,
                   j->p->d + r * t->nb, j->p->m + r * t->nb);
        block_sums(j->p->q + r * t->k, t->nb, j->p->sum + r * t->nb);
    }
    return NULL;
}

/* quant.rs:589-639 */
static packed_t *packed_i8(cb_qtensor *t, int threads)
{
    pthread_mutex_lock(&t->lock);
    if (!t->packed) {
        packed_t *p = (packed_t *)calloc(1, sizeof(*p));
        p->q = (int8_t *)malloc(t->n * t->k);
        p->d = (float *)malloc(t->n * t->nb * sizeof(float));
        p->m = (float *)malloc(t->n * t->nb * sizeof(float));
        p->sum = (int32_t *)malloc(t->n * t->nb * sizeof(int32_t));
        if (threads > 1 && t->n > (size_t)threads) {
            size_t chunk = (t->n + threads - 1) / threads;
            size_t nj = (t->n + chunk - 1) / chunk;
            pthread_t *th = (pthread_t *)malloc(nj * sizeof(pthread_t));
            pack_job_t *jobs = (pack_job_t *)malloc(nj * sizeof(pack_job_t));
            for (size_t c = 0; c < nj; c++) {
                jobs[c].t = t;
                jobs[c].p = p;
                jobs[c].r0 = c * chunk;
                jobs[c].r1 = (c + 1) * chunk < t->n ? (c + 1) * chunk : t->n;
                pthread_create(&th[c], NULL, pack_rows, &jobs[c]);
            }
            for (size_t c = 0; c < nj; c++)
                pthread_join(th[c], NULL);
            free(th);
            free(jobs);
        } else {
            pack_job_t j = {t, p, 0, t->n};
            pack_rows(&j);
        }
        t->packed = p;
    }
    pthread_mutex_unlock(&t->lock);
    return t->packed;
}

/* ---------------------------------------------------------- matmul */

typedef struct {
    const cb_qtensor *b;
    const float *a;
    size_t m;
    const int8_t *qa;
    const float *da;
    const int32_t *sa;
    const packed_t *packed;
    int tier;
    size_t j0, cols;
    float *buf; /* [m, cols] */
} cols_job_t;

static void run_rows(const cols_job_t *c, size_t m0, size_t m1, size_t jb, size_t jn,
                     const int8_t *qb, const float *db, const float *mb, const int32_t *sumb,
                     size_t qstride, size_t sstride)
{
    size_t k = c->b->k, nb = c->b->nb;
    size_t i = m0;
    while (i < m1) {
        int nr = (m1 - i >= 4) ? 4 : 1; /* x4 groups, then single rows */
        rows4_t rows;
        for (int r = 0; r < nr; r++) {
            rows.q[r] = c->qa + (i + r) * k;
            rows.d[r] = c->da + (i + r) * nb;
            rows.s[r] = c->sa + (i + r) * nb;
        }
        for (size_t r = 0; r < jn; r++) {
            float o[4];
            if (c->tier == TIER_VNNI)
                dot_vnni_x4(&rows, nr, qb + r * qstride, db + r * sstride, mb + r * sstride,
                            sumb + r * sstride, nb, o);
            else
                dot_avx2_x4(&rows, nr, qb + r * qstride, db + r * sstride, mb + r * sstride, nb, o);
            for (int rr = 0; rr < nr; rr++)
                c->buf[(i + rr) * c->cols + (jb + r - c->j0)] = o[rr];
        }
        i += (size_t)nr;
    }
}

/* the body of quant.rs:790-1019 (`cols_block`) */
static void *cols_block(void *arg)
{
    cols_job_t *c = (cols_job_t *)arg;
    const cb_qtensor *b = c->b;
    size_t m = c->m, k = b->k, nb = b->nb;
    if (c->tier == TIER_F32) { /* quant.rs:995-1018 */
        float *fb = (float *)malloc(k * sizeof(float));
        for (size_t j = c->j0; j < c->j0 + c->cols; j++) {
            or_dequant_row(b->dtype, b->raw + j * nb * (size_t)b->bb, nb, fb);
            for (size_t i = 0; i < m; i++) {
                float out;
                or_matmul_t_dense(c->a + i * k, 1, k, fb, 1, &out);
                c->buf[i * c->cols + (j - c->j0)] = out;
            }
        }
        free(fb);
        return NULL;
    }
    if (c->packed) {
        const packed_t *p = c->packed;
        for (size_t m0 = 0; m0 < m; m0 += M_BLOCK) {
            size_t m1 = m0 + M_BLOCK < m ? m0 + M_BLOCK : m;
            for (size_t j = c->j0; j < c->j0 + c->cols; j += N_BLOCK) {
                size_t jn = c->j0 + c->cols - j < N_BLOCK ? c->j0 + c->cols - j : N_BLOCK;
                run_rows(c, m0, m1, j, jn, p->q + j * k, p->d + j * nb, p->m + j * nb,
                         p->sum + j * nb, k, nb);
            }
        }
        return NULL;
    }
    int8_t *qb = (int8_t *)malloc(N_BLOCK * k);
    float *db = (float *)malloc(N_BLOCK * nb * sizeof(float));
    float *mb = (float *)malloc(N_BLOCK * nb * sizeof(float));
    int32_t *sumb = (int32_t *)calloc(N_BLOCK * nb, sizeof(int32_t));
    for (size_t m0 = 0; m0 < m; m0 += M_BLOCK) {
        size_t m1 = m0 + M_BLOCK < m ? m0 + M_BLOCK : m;
        for (size_t j = c->j0; j < c->j0 + c->cols; j += N_BLOCK) {
            size_t jn = c->j0 + c->cols - j < N_BLOCK ? c->j0 + c->cols - j : N_BLOCK;
            for (size_t r = 0; r < jn; r++) {
                unpack_row(b->dtype, b->raw + (j + r) * nb * (size_t)b->bb, b->bb, nb, qb + r * k,
                           db + r * nb, mb + r * nb);
                if (c->tier == TIER_VNNI)
                    block_sums(qb + r * k, nb, sumb + r * nb);
            }
            run_rows(c, m0, m1, j, jn, qb, db, mb, sumb, k, nb);
        }
    }
    free(qb);
    free(db);
    free(mb);
    free(sumb);
    return NULL;
}

/* quant.rs:754-1051 (+ linear_w's bias, quant.rs:1054-1063).  tier < 0
 * selects by CPU detection; threads <= 0 uses available_parallelism. */
int cb_matmul_t_q(const float *a, size_t m, cb_qtensor *b, const float *bias, float *out, int tier,
                  int threads, int *tier_used)
{
    if (!b || !a || !out)
        return -1;
    size_t k = b->k, n = b->n, nb = b->nb;
    int det = cb_detect_tier();
    if (tier < 0)
        tier = det;
    if (tier < det) /* asked for an ISA this CPU does not have */
        return -2;
    if (threads <= 0)
        threads = cb_hw_threads();
    if (tier_used)
        *tier_used = tier;

    int8_t *qa = NULL;
    float *da = NULL;
    int32_t *sa = NULL;
    const packed_t *packed = NULL;
    if (tier != TIER_F32) {
        qa = (int8_t *)malloc(m * k + 1);
        da = (float *)malloc(m * nb * sizeof(float) + 4);
        sa = (int32_t *)malloc(m * nb * sizeof(int32_t) + 4);
        or_quantize_acts(a, m, k, qa, da, sa);
        pthread_mutex_lock(&b->lock);
        size_t prior = b->calls++;
        pthread_mutex_unlock(&b->lock);
        if (prior >= 1)
            packed = packed_i8(b, threads);
    }

    if (threads > 1 && (double)m * (double)n * (double)k > (double)PAR_THRESHOLD) {
        size_t chunk = (n + threads - 1) / threads;
        size_t nj = (n + chunk - 1) / chunk;
        pthread_t *th = (pthread_t *)malloc(nj * sizeof(pthread_t));
        cols_job_t *jobs = (cols_job_t *)malloc(nj * sizeof(cols_job_t));
        for (size_t c = 0; c < nj; c++) {
            size_t j0 = c * chunk;
            size_t cols = chunk < n - j0 ? chunk : n - j0;
            cols_job_t jb = {b, a, m, qa, da, sa, packed, tier, j0, cols,
                             (float *)malloc(m * cols * sizeof(float) + 4)};
            jobs[c] = jb;
            pthread_create(&th[c], NULL, cols_block, &jobs[c]);
        }
        for (size_t c = 0; c < nj; c++)
            pthread_join(th[c], NULL);
        for (size_t c = 0; c < nj; c++) { /* serial copy-back, quant.rs:1039-1044 */
            for (size_t i = 0; i < m; i++)
                memcpy(out + i * n + jobs[c].j0, jobs[c].buf + i * jobs[c].cols,
                       jobs[c].cols * sizeof(float));
            free(jobs[c].buf);
        }
        free(th);
        free(jobs);
    } else {
        float *buf = (float *)malloc(m * n * sizeof(float) + 4);
        cols_job_t jb = {b, a, m, qa, da, sa, packed, tier, 0, n, buf};
        cols_block(&jb);
        memcpy(out, buf, m * n * sizeof(float));
        free(buf);
    }
    if (bias) /* tensor.rs:263-271 */
        for (size_t i = 0; i < m; i++)
            for (size_t j = 0; j < n; j++)
                out[i * n + j] = out[i * n + j] + bias[j];
    free(qa);
    free(da);
    free(sa);
    return 0;
}
