/*
 * oracle.h -- CPU restatement of rusty_whisper's quantized linear-layer
 * matmul (src/quant.rs), used ONLY as test infrastructure: the parity
 * reference for tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg.  Nothing in the product (rusty_whisper_amd/, include/) links or calls
 * this code.
 *
 * Every function cites the reference file:line it restates.  Pinning (what
 * checks each function against something other than itself) is listed per
 * function; a function with no such check would say "parity unpinned" -- none
 * does at present:
 *
 *   or_f16_to_f32 / or_f32_to_f16   model.rs KATs (model.rs:282-291,
 *                                   model.rs:391-398) + exhaustive 65536-code
 *                                   sweep against numpy.float16 (finite codes)
 *   or_unpack_block / or_dequant    hand-built block KATs (model.rs:348-381,
 *                                   quant.rs:1162-1174, model.rs:412-416) +
 *                                   closed form x = d*q + m over every nibble /
 *                                   high-bit pattern
 *   or_quantize_acts                closed-form edge vectors (zero block,
 *                                   exact halves, +-amax, NaN/inf, subnormal d)
 *                                   + an independent numpy float32 restatement
 *   or_block_dots                   int64 brute force in numpy
 *   or_matmul_emul (VNNI / AVX2)    bitwise against the intrinsics port in
 *                                   cpu_baseline.c on this AVX-512 VNNI host;
 *                                   reference tolerances vs dense-on-dequant
 *                                   (quant.rs:1187-1301) and vs the scalar
 *                                   int8 reference (quant.rs:1336-1370)
 *   or_matmul_exact                 float64 of the exact integer sums;
 *                                   checked against numpy float64 matmul of the
 *                                   dequantized operands
 *   or_matmul_t_dense               tensor.rs KATs (tensor.rs:376-471 style
 *                                   small cases) + numpy float64 matmul
 *   quantizers / or_test_matrix     LCG closed form (quant.rs:1115-1123);
 *                                   encode->decode error bounds per format
 */
#ifndef RW_ORACLE_H
#define RW_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_QK 32

/* model.rs:68-86 */
float or_f16_to_f32(uint16_t h);
/* model.rs:68-86 over an array (bits never pass through a double) */
void or_f16_to_f32_array(const uint16_t *h, size_t n, float *out);
/* model.rs:90-115 (round-half-up on the first dropped bit, not IEEE RNE) */
uint16_t or_f32_to_f16(float x);

/* quant.rs:43-52; -1 for an unsupported dtype */
int or_block_bytes(int dtype);

/* quant.rs:98-131: one block -> 32 centered int8 + (d, m); returns 0 or -1 */
int or_unpack_block(int dtype, const uint8_t *block, int8_t *q, float *d, float *m);

/* quant.rs:528-537: nblocks consecutive blocks -> nblocks*32 f32 */
int or_dequant_row(int dtype, const uint8_t *raw, size_t nblocks, float *out);

/* quant.rs:691-716: activations [m,k] -> q[m*k] (natural element order),
 * d[m*nb], sum[m*nb] */
void or_quantize_acts(const float *a, size_t m, size_t k, int8_t *q, float *d, int32_t *sum);

/* quant.rs:256-320 + quant.rs:403-418: weight row -> qb[k], db/mb[nb], sumb[nb] */
int or_unpack_row_i8(int dtype, const uint8_t *raw, size_t nb, int8_t *qb, float *db,
                     float *mb, int32_t *sumb);

/* Exact per-block integer dot sums S[i][j][bl] = sum_e qa[i,bl*32+e]*qb[j,bl*32+e]
 * (the integer inner product of quant.rs:1-13, 330-490).  S is [m][n][nb]. */
int or_block_dots(int dtype, const uint8_t *raw, size_t n, size_t k, const int8_t *qa, size_t m,
                  int32_t *S);

/* Lane-exact scalar emulation of matmul_t_q's int8 tier.
 *   tier 0: AVX-512 VNNI kernels (quant.rs:429-490)
 *   tier 1: AVX2 maddubs kernels (quant.rs:330-395)
 * Output is bitwise what the reference produces on such a host: the f32
 * accumulation follows the 8-lane layout, hsum256_ps (quant.rs:242-247) and
 * the scalar `corr` order.  out is [m][n]; bias (may be NULL) is added after
 * as add_bias (tensor.rs:263-271, via linear_w quant.rs:1054-1063). */
int or_matmul_emul(int tier, const float *a, size_t m, size_t k, int dtype, const uint8_t *raw,
                   size_t n, const float *bias, float *out);

/* Same math with the exact integer sums combined in float64:
 * out = sum_bl d_a*d_b*S + m_b*d_a*sum_a (+ bias).  The "truth" the f32
 * paths are measured against. */
int or_matmul_exact(const float *a, size_t m, size_t k, int dtype, const uint8_t *raw, size_t n,
                    const float *bias, double *out);

/* tensor.rs:110-158 + tensor.rs:194-238: f32 C = A B^T with the 8-lane dot
 * (the dense-on-dequant reference the quant.rs tests compare against). */
void or_matmul_t_dense(const float *a, size_t m, size_t k, const float *b, size_t n, float *out);

/* quant.rs:1115-1123: the tests' LCG matrix generator */
void or_test_matrix(size_t count, uint32_t seed, float *out);

/* quant.rs:1071-1083 and quant.rs:1088-1113: the tests' quantizers.  Q4_0,
 * Q4_1 and Q5_0 have no quantizer in the reference; ours produce valid ggml
 * blocks (any valid encoder is acceptable: the bytes are inputs). Each
 * returns the byte count written (count/32 blocks). */
size_t or_quantize(int dtype, const float *x, size_t count, uint8_t *raw);

#ifdef __cplusplus
}
#endif
#endif
