/*
 * oracle.c -- CPU restatement of rusty_whisper src/quant.rs (and the f16
 * codec of src/model.rs, the f32 dot of src/tensor.rs) for the quantized
 * linear-layer matmul.  TEST INFRASTRUCTURE ONLY: the reference values for tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg.  The product
 * (rusty_whisper_amd/, include/) never links or calls it.
 *
 * Must be compiled with -ffp-contract=off and without -ffast-math: the
 * reference is Rust, which never contracts a*b+c into an FMA, and the lane
 * emulations below reproduce its exact f32 rounding sequence.  Where the
 * reference does use an FMA (_mm256_fmadd_ps) we call fmaf explicitly.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ f16 */

/* model.rs:68-86 */
float or_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15);
    uint32_t exp = (uint32_t)((h >> 10) & 0x1f);
    uint32_t frac = (uint32_t)(h & 0x3ff);
    uint32_t bits;
    if (exp == 0 && frac == 0) {
        bits = sign << 31;
    } else if (exp == 0) {
        /* subnormal: value = frac * 2^-24; the msb at position p becomes the
         * implicit bit, giving unbiased exponent p - 24 */
        uint32_t p = 31u - (uint32_t)__builtin_clz(frac);
        uint32_t mant = (frac << (10u - p)) & 0x3ffu;
        bits = (sign << 31) | ((p + 103u) << 23) | (mant << 13);
    } else if (exp == 0x1f && frac == 0) {
        bits = (sign << 31) | 0x7f800000u;
    } else if (exp == 0x1f) {
        bits = (sign << 31) | 0x7f800000u | (frac << 13);
    } else {
        bits = (sign << 31) | ((exp + 127u - 15u) << 23) | (frac << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void or_f16_to_f32_array(const uint16_t *h, size_t n, float *out)
{
    for (size_t i = 0; i < n; i++)
        out[i] = or_f16_to_f32(h[i]);
}

/* model.rs:90-115 */
uint16_t or_f32_to_f16(float x)
{
    uint32_t bits;
    memcpy(&bits, &x, 4);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    int32_t exp = (int32_t)((bits >> 23) & 0xffu);
    uint32_t frac = bits & 0x007fffffu;
    if (exp == 0xff)
        return (uint16_t)(sign | 0x7c00u | (frac != 0 ? 0x200u : 0u));
    int32_t e = exp - 127 + 15;
    if (e >= 0x1f)
        return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10)
            return sign;
        uint32_t f = frac | 0x00800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint16_t half = (uint16_t)(f >> shift);
        uint16_t round = (uint16_t)((f >> (shift - 1)) & 1u);
        return (uint16_t)(sign | (uint16_t)(half + round));
    }
    uint16_t half = (uint16_t)((((uint32_t)e) << 10) | (frac >> 13));
    uint16_t round = (uint16_t)((frac >> 12) & 1u);
    return (uint16_t)(sign | (uint16_t)(half + round));
}

static float half_at(const uint8_t *p) { return or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

static uint32_t u32_at(const uint8_t *p)
{
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* ---------------------------------------------------------- block codec */

/* quant.rs:43-52 */
int or_block_bytes(int dtype)
{
    switch (dtype) {
    case 2: return 18; /* Q4_0 */
    case 3: return 20; /* Q4_1 */
    case 6: return 22; /* Q5_0 */
    case 7: return 24; /* Q5_1 */
    case 8: return 34; /* Q8_0 */
    default: return -1;
    }
}

/* quant.rs:57-63: low nibble -> element j, high nibble -> element j+16 */
static void unpack_nibbles(const uint8_t *packed, int8_t *q, int offset)
{
    for (int j = 0; j < OR_QK / 2; j++) {
        q[j] = (int8_t)((packed[j] & 0x0f) - offset);
        q[j + OR_QK / 2] = (int8_t)((packed[j] >> 4) - offset);
    }
}

/* quant.rs:69-94: qh bit j adds 16 to element j (the HI_BITS table is a
 * lookup form of exactly this) */
static void apply_high_bits(uint32_t qh, int8_t *q)
{
    for (int j = 0; j < OR_QK; j++)
        q[j] = (int8_t)(q[j] + (int8_t)(((qh >> j) & 1u) << 4));
}

/* quant.rs:98-131 */
int or_unpack_block(int dtype, const uint8_t *block, int8_t *q, float *d, float *m)
{
    switch (dtype) {
    case 2:
        unpack_nibbles(block + 2, q, 8);
        *d = half_at(block);
        *m = 0.0f;
        return 0;
    case 3:
        unpack_nibbles(block + 4, q, 0);
        *d = half_at(block);
        *m = half_at(block + 2);
        return 0;
    case 6: {
        uint32_t qh = u32_at(block + 2);
        unpack_nibbles(block + 6, q, 0);
        apply_high_bits(qh, q);
        for (int j = 0; j < OR_QK; j++)
            q[j] = (int8_t)(q[j] - 16);
        *d = half_at(block);
        *m = 0.0f;
        return 0;
    }
    case 7: {
        uint32_t qh = u32_at(block + 4);
        unpack_nibbles(block + 8, q, 0);
        apply_high_bits(qh, q);
        *d = half_at(block);
        *m = half_at(block + 2);
        return 0;
    }
    case 8:
        for (int j = 0; j < OR_QK; j++)
            q[j] = (int8_t)block[2 + j];
        *d = half_at(block);
        *m = 0.0f;
        return 0;
    default:
        return -1;
    }
}

/* quant.rs:528-537: o[l] = d * q[l] as f32 + m (mul, then add) */
int or_dequant_row(int dtype, const uint8_t *raw, size_t nblocks, float *out)
{
    int bb = or_block_bytes(dtype);
    if (bb < 0)
        return -1;
    int8_t q[OR_QK];
    for (size_t b = 0; b < nblocks; b++) {
        float d, m;
        or_unpack_block(dtype, raw + b * (size_t)bb, q, &d, &m);
        for (int l = 0; l < OR_QK; l++) {
            float p = d * (float)q[l];
            out[b * OR_QK + l] = p + m;
        }
    }
    return 0;
}

/* ------------------------------------------------- activation quantizer */

/* Rust f32::max / f32::min return the non-NaN operand, as fmaxf/fminf do. */

/* Rust `(v * inv).round().clamp(-127.0, 127.0) as i32`: round half away
 * from zero, clamp keeps NaN, `as i32` maps NaN to 0. */
static int32_t round_clamp_i8(float v)
{
    float r = roundf(v);
    if (r != r)
        return 0;
    if (r < -127.0f)
        r = -127.0f;
    if (r > 127.0f)
        r = 127.0f;
    return (int32_t)r;
}

/* quant.rs:691-716 */
void or_quantize_acts(const float *a, size_t m, size_t k, int8_t *q, float *d, int32_t *sum)
{
    size_t nb = k / OR_QK;
    for (size_t i = 0; i < m; i++) {
        for (size_t bl = 0; bl < nb; bl++) {
            const float *x = a + i * k + bl * OR_QK;
            float amax = 0.0f;
            for (int l = 0; l < OR_QK; l++)
                amax = fmaxf(amax, fabsf(x[l]));
            float dd = amax / 127.0f;
            float inv = dd > 0.0f ? 1.0f / dd : 0.0f;
            int32_t s = 0;
            for (int l = 0; l < OR_QK; l++) {
                int32_t qq = round_clamp_i8(x[l] * inv);
                q[i * k + bl * OR_QK + l] = (int8_t)qq;
                s += qq;
            }
            d[i * nb + bl] = dd;
            sum[i * nb + bl] = s;
        }
    }
}

/* ---------------------------------------------------- weight unpacking */

/* quant.rs:256-320 (row -> i8 + per-block d/m) and quant.rs:403-418 (sumb) */
int or_unpack_row_i8(int dtype, const uint8_t *raw, size_t nb, int8_t *qb, float *db, float *mb,
                     int32_t *sumb)
{
    int bb = or_block_bytes(dtype);
    if (bb < 0)
        return -1;
    for (size_t bl = 0; bl < nb; bl++) {
        or_unpack_block(dtype, raw + bl * (size_t)bb, qb + bl * OR_QK, &db[bl], &mb[bl]);
        if (sumb) {
            int32_t s = 0;
            for (int l = 0; l < OR_QK; l++)
                s += qb[bl * OR_QK + l];
            sumb[bl] = s;
        }
    }
    return 0;
}

typedef struct {
    int8_t *q;
    float *d;
    float *m;
    int32_t *sum;
} unpacked_t;

static int unpack_matrix(int dtype, const uint8_t *raw, size_t n, size_t k, unpacked_t *u)
{
    int bb = or_block_bytes(dtype);
    if (bb < 0 || k % OR_QK)
        return -1;
    size_t nb = k / OR_QK;
    u->q = (int8_t *)malloc(n * k);
    u->d = (float *)malloc(n * nb * sizeof(float));
    u->m = (float *)malloc(n * nb * sizeof(float));
    u->sum = (int32_t *)malloc(n * nb * sizeof(int32_t));
    if (!u->q || !u->d || !u->m || !u->sum)
        return -1;
    for (size_t j = 0; j < n; j++)
        or_unpack_row_i8(dtype, raw + j * nb * (size_t)bb, nb, u->q + j * k, u->d + j * nb,
                         u->m + j * nb, u->sum + j * nb);
    return 0;
}

static void unpacked_free(unpacked_t *u)
{
    free(u->q);
    free(u->d);
    free(u->m);
    free(u->sum);
}

typedef struct {
    int8_t *q;
    float *d;
    int32_t *sum;
} qacts_t;

static int qacts_make(const float *a, size_t m, size_t k, qacts_t *qa)
{
    size_t nb = k / OR_QK;
    qa->q = (int8_t *)malloc(m * k + 1);
    qa->d = (float *)malloc(m * nb * sizeof(float) + 4);
    qa->sum = (int32_t *)malloc(m * nb * sizeof(int32_t) + 4);
    if (!qa->q || !qa->d || !qa->sum)
        return -1;
    or_quantize_acts(a, m, k, qa->q, qa->d, qa->sum);
    return 0;
}

static void qacts_free(qacts_t *qa)
{
    free(qa->q);
    free(qa->d);
    free(qa->sum);
}

/* ------------------------------------------------------ exact int sums */

int or_block_dots(int dtype, const uint8_t *raw, size_t n, size_t k, const int8_t *qa, size_t m,
                  int32_t *S)
{
    unpacked_t u;
    if (unpack_matrix(dtype, raw, n, k, &u))
        return -1;
    size_t nb = k / OR_QK;
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++)
            for (size_t bl = 0; bl < nb; bl++) {
                const int8_t *x = qa + i * k + bl * OR_QK;
                const int8_t *y = u.q + j * k + bl * OR_QK;
                int32_t s = 0;
                for (int l = 0; l < OR_QK; l++)
                    s += (int32_t)x[l] * (int32_t)y[l];
                S[(i * n + j) * nb + bl] = s;
            }
    unpacked_free(&u);
    return 0;
}

/* ------------------------------------------------ lane-exact emulations */

/* quant.rs:242-247: lo128 + hi128, then two hadds */
static float hsum256(const float acc[8])
{
    float s0 = acc[0] + acc[4];
    float s1 = acc[1] + acc[5];
    float s2 = acc[2] + acc[6];
    float s3 = acc[3] + acc[7];
    float h0 = s0 + s1;
    float h1 = s2 + s3;
    return h0 + h1;
}

/* quant.rs:468-490 (dot_i8_vnni; the x4 form at quant.rs:431-460 performs the
 * identical per-row operation sequence) */
static float dot_vnni(const int8_t *qa, const float *da, const int32_t *suma, const int8_t *qb,
                      const float *db, const float *mb, const int32_t *sumb, size_t nb)
{
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float corr = 0.0f;
    for (size_t bl = 0; bl < nb; bl++) {
        const int8_t *x = qa + bl * OR_QK;
        const int8_t *y = qb + bl * OR_QK;
        float s = da[bl] * db[bl];
        for (int t = 0; t < 8; t++) {
            /* dpbusd: u8 (q_a + 128, the xor with 0x80) times i8 q_b, four
             * adjacent bytes into one i32 lane */
            int32_t dp = 0;
            for (int u = 0; u < 4; u++)
                dp += (int32_t)(uint8_t)(x[4 * t + u] ^ 0x80) * (int32_t)y[4 * t + u];
            acc[t] = fmaf(s, (float)dp, acc[t]);
        }
        float c1 = s * -128.0f;
        c1 = c1 * (float)sumb[bl];
        float c2 = mb[bl] * da[bl];
        c2 = c2 * (float)suma[bl];
        corr = corr + (c1 + c2);
    }
    return hsum256(acc) + corr;
}

/* quant.rs:331-354 (dot_i8_avx2; x4 form quant.rs:366-395 is identical per row) */
static float dot_avx2(const int8_t *qa, const float *da, const int32_t *suma, const int8_t *qb,
                      const float *db, const float *mb, size_t nb)
{
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float corr = 0.0f;
    for (size_t bl = 0; bl < nb; bl++) {
        const int8_t *x = qa + bl * OR_QK;
        const int8_t *y = qb + bl * OR_QK;
        float scale = da[bl] * db[bl];
        for (int t = 0; t < 8; t++) {
            /* maddubs(|b|, sign(a,b)) then madd(.,1): lane t sums the four
             * exact products of elements 4t..4t+3 (no i16 saturation: every
             * pair sum is at most 2*128*127) */
            int32_t p = 0;
            for (int u = 0; u < 4; u++)
                p += (int32_t)x[4 * t + u] * (int32_t)y[4 * t + u];
            acc[t] = fmaf(scale, (float)p, acc[t]);
        }
        float c = mb[bl] * da[bl];
        c = c * (float)suma[bl];
        corr = corr + c;
    }
    return hsum256(acc) + corr;
}

int or_matmul_emul(int tier, const float *a, size_t m, size_t k, int dtype, const uint8_t *raw,
                   size_t n, const float *bias, float *out)
{
    if (k % OR_QK || or_block_bytes(dtype) < 0 || (tier != 0 && tier != 1))
        return -1;
    size_t nb = k / OR_QK;
    unpacked_t u;
    qacts_t qa;
    if (unpack_matrix(dtype, raw, n, k, &u))
        return -1;
    if (qacts_make(a, m, k, &qa)) {
        unpacked_free(&u);
        return -1;
    }
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            float v;
            if (tier == 0)
                v = dot_vnni(qa.q + i * k, qa.d + i * nb, qa.sum + i * nb, u.q + j * k,
                             u.d + j * nb, u.m + j * nb, u.sum + j * nb, nb);
            else
                v = dot_avx2(qa.q + i * k, qa.d + i * nb, qa.sum + i * nb, u.q + j * k,
                             u.d + j * nb, u.m + j * nb, nb);
            if (bias)
                v = v + bias[j];
            out[i * n + j] = v;
        }
    qacts_free(&qa);
    unpacked_free(&u);
    return 0;
}

int or_matmul_exact(const float *a, size_t m, size_t k, int dtype, const uint8_t *raw, size_t n,
                    const float *bias, double *out)
{
    if (k % OR_QK || or_block_bytes(dtype) < 0)
        return -1;
    size_t nb = k / OR_QK;
    unpacked_t u;
    qacts_t qa;
    if (unpack_matrix(dtype, raw, n, k, &u))
        return -1;
    if (qacts_make(a, m, k, &qa)) {
        unpacked_free(&u);
        return -1;
    }
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            double acc = 0.0;
            for (size_t bl = 0; bl < nb; bl++) {
                const int8_t *x = qa.q + i * k + bl * OR_QK;
                const int8_t *y = u.q + j * k + bl * OR_QK;
                int64_t s = 0;
                for (int l = 0; l < OR_QK; l++)
                    s += (int64_t)x[l] * (int64_t)y[l];
                double da = qa.d[i * nb + bl];
                acc += da * (double)u.d[j * nb + bl] * (double)s +
                       (double)u.m[j * nb + bl] * da * (double)qa.sum[i * nb + bl];
            }
            if (bias)
                acc += (double)bias[j];
            out[i * n + j] = acc;
        }
    qacts_free(&qa);
    unpacked_free(&u);
    return 0;
}

/* --------------------------------------------------------- dense f32 */

/* tensor.rs:110-129: 8 per-lane accumulators, mul then add; the lane sum
 * and the tail are `Iterator::sum` folds (which start from -0.0) */
static float dot8(const float *a, const float *b, size_t k)
{
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t k8 = k / 8 * 8;
    for (size_t p = 0; p < k8; p += 8)
        for (int l = 0; l < 8; l++) {
            float prod = a[p + l] * b[p + l];
            acc[l] = acc[l] + prod;
        }
    float tail = -0.0f;
    for (size_t p = k8; p < k; p++) {
        float prod = a[p] * b[p];
        tail = tail + prod;
    }
    float s = -0.0f;
    for (int l = 0; l < 8; l++)
        s = s + acc[l];
    return s + tail;
}

/* tensor.rs:194-238 (dot4 at tensor.rs:132-158 is dot8 per row) */
void or_matmul_t_dense(const float *a, size_t m, size_t k, const float *b, size_t n, float *out)
{
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++)
            out[i * n + j] = dot8(a + i * k, b + j * k, k);
}

/* ------------------------------------------------------ test helpers */

/* quant.rs:1115-1123 */
void or_test_matrix(size_t count, uint32_t seed, float *out)
{
    uint32_t state = seed;
    for (size_t i = 0; i < count; i++) {
        state = state * 1664525u + 1013904223u;
        float v = (float)(state >> 8) / 16777216.0f;
        v = v * 2.0f;
        out[i] = v - 1.0f;
    }
}

static void put_f16(uint8_t *p, float v)
{
    uint16_t h = or_f32_to_f16(v);
    p[0] = (uint8_t)(h & 0xff);
    p[1] = (uint8_t)(h >> 8);
}

static void put_u32(uint8_t *p, uint32_t v)
{
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
    p[2] = (uint8_t)(v >> 16);
    p[3] = (uint8_t)(v >> 24);
}

/* Rust `x.round().clamp(lo, hi) as u8` (saturating cast, NaN -> 0) */
static uint8_t round_clamp_u8(float v, float hi)
{
    float r = roundf(v);
    if (r != r)
        return 0;
    if (r < 0.0f)
        r = 0.0f;
    if (r > hi)
        r = hi;
    return (uint8_t)r;
}

/* the element of largest magnitude, sign kept */
static float signed_absmax(const float *x)
{
    float amax = 0.0f, vmax = 0.0f;
    for (int l = 0; l < OR_QK; l++)
        if (fabsf(x[l]) > amax) {
            amax = fabsf(x[l]);
            vmax = x[l];
        }
    return vmax;
}

static void pack_nibbles(const uint8_t *qs, uint8_t *out)
{
    for (int e = 0; e < 16; e++)
        out[e] = (uint8_t)((qs[e] & 0x0f) | ((qs[e + 16] & 0x0f) << 4));
}

static uint32_t high_bits_of(const uint8_t *qs)
{
    uint32_t qh = 0;
    for (int e = 0; e < OR_QK; e++)
        if (qs[e] & 0x10)
            qh |= 1u << e;
    return qh;
}

size_t or_quantize(int dtype, const float *x, size_t count, uint8_t *raw)
{
    int bb = or_block_bytes(dtype);
    if (bb < 0 || count % OR_QK)
        return 0;
    size_t nblk = count / OR_QK;
    for (size_t b = 0; b < nblk; b++) {
        const float *blk = x + b * OR_QK;
        uint8_t *o = raw + b * (size_t)bb;
        uint8_t qs[OR_QK];
        switch (dtype) {
        case 8: { /* quant.rs:1071-1083 */
            float amax = 0.0f;
            for (int l = 0; l < OR_QK; l++)
                amax = fmaxf(amax, fabsf(blk[l]));
            float d = amax / 127.0f;
            float id = d > 0.0f ? 1.0f / d : 0.0f;
            put_f16(o, d);
            for (int l = 0; l < OR_QK; l++)
                o[2 + l] = (uint8_t)(int8_t)round_clamp_i8(blk[l] * id);
            break;
        }
        case 7: { /* quant.rs:1088-1113 */
            float mn = 3.40282347e38f, mx = -3.40282347e38f;
            for (int l = 0; l < OR_QK; l++) {
                mn = fminf(mn, blk[l]);
                mx = fmaxf(mx, blk[l]);
            }
            float d = (mx - mn) / 31.0f;
            float id = d > 0.0f ? 1.0f / d : 0.0f;
            for (int l = 0; l < OR_QK; l++)
                qs[l] = round_clamp_u8((blk[l] - mn) * id, 31.0f);
            put_f16(o, d);
            put_f16(o + 2, mn);
            put_u32(o + 4, high_bits_of(qs));
            pack_nibbles(qs, o + 8);
            break;
        }
        case 3: { /* Q4_1: asymmetric 4-bit, 15 steps between min and max */
            float mn = 3.40282347e38f, mx = -3.40282347e38f;
            for (int l = 0; l < OR_QK; l++) {
                mn = fminf(mn, blk[l]);
                mx = fmaxf(mx, blk[l]);
            }
            float d = (mx - mn) / 15.0f;
            float id = d > 0.0f ? 1.0f / d : 0.0f;
            for (int l = 0; l < OR_QK; l++)
                qs[l] = round_clamp_u8((blk[l] - mn) * id, 15.0f);
            put_f16(o, d);
            put_f16(o + 2, mn);
            pack_nibbles(qs, o + 4);
            break;
        }
        case 2: { /* Q4_0: symmetric, the extreme element maps to code 0 (-8) */
            float vmax = signed_absmax(blk);
            float d = vmax / -8.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            for (int l = 0; l < OR_QK; l++)
                qs[l] = round_clamp_u8(blk[l] * id + 8.0f, 15.0f);
            put_f16(o, d);
            pack_nibbles(qs, o + 2);
            break;
        }
        case 6: { /* Q5_0: symmetric 5-bit, extreme element maps to code 0 (-16) */
            float vmax = signed_absmax(blk);
            float d = vmax / -16.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            for (int l = 0; l < OR_QK; l++)
                qs[l] = round_clamp_u8(blk[l] * id + 16.0f, 31.0f);
            put_f16(o, d);
            put_u32(o + 2, high_bits_of(qs));
            pack_nibbles(qs, o + 6);
            break;
        }
        }
    }
    return nblk * (size_t)bb;
}
