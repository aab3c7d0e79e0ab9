// rw_layout.hpp -- how quantized weights and quantized activations sit in HBM.
//
// Weights ([n, k] ggml matrix, nb = k/32 blocks per row) are repacked once at
// upload into the decode / validation planes below and the GEMM planes.
// Rows are interleaved in groups of 32 ("row groups"), so the 32 rows of one
// group are contiguous for a given block:
// a wavefront reading one block of 32 consecutive rows touches one
// contiguous span.  Blocks are padded to a multiple of 8 ("octets") so the
// per-block scalars of 8 blocks are 16/32 contiguous bytes per row.
//
//   qs  [ngroups][nb_pad][32 rows][QSB]   QSB = 16 (Q4/Q5: packed nibbles,
//        byte t = element t | element t+16 << 4, as in ggml) or 32 (Q8_0:
//        int8 in MFMA order, see below)
//   qh  [ngroups][noct][32 rows][8 blocks] u32, Q5 only, bit-permuted (below)
//   d   [ngroups][noct][32 rows][8 blocks] f16 bits (block scale)
//   m   [ngroups][noct][32 rows][8 blocks] f16 bits (block min, _1 formats)
//
// Rows past n and blocks past nb are zero (d = m = 0), so they contribute
// nothing.
//
// MFMA order.  One v_mfma_i32_32x32x32_i8 consumes one 32-element block per
// operand row: lane l supplies row l%32, and lane half h = l/32 supplies 16
// of the 32 elements.  Any assignment of elements to (h, byte) works as long
// as activations and weights use the same one; we use
//     h = 0: elements 0-7 then 16-23,   h = 1: elements 8-15 then 24-31
// because that is what 8 packed nibble bytes qs[8h..8h+8) give directly
// (low nibbles = elements 8h.., high nibbles = elements 16+8h..).  Stored
// 32-byte blocks (Q8_0 weights, quantized activations) are kept in that order:
//     position p holds element  p (p<8), p+8 (8<=p<16), p-8 (16<=p<24), p (p>=24)
// (the map is its own inverse).
//
// High bits.  A Q5 block's 32 high bits are stored permuted so that the
// flag word of "natural dword" t (elements 4t..4t+3, one per byte) is
// rotl(X, t) & 0x10101010: element 4t+u's bit sits at bit (8u + 4 - t) mod 32
// of X.  Two VALU ops per 4 elements instead of four.
//
// GEMM planes (weights), indexed like qs:
//   q8  [ngroups][nb_pad][32 rows][32 B]  every quant as one byte in MFMA
//        order (Q4/Q5 the unsigned value as stored; Q8_0 reads qs itself)
//   dm  [ngroups][nb_pad][32 rows]        u32: f16 d_b (low), f16 m_b - cm
//        (high), both divided by the row's power-of-two scale cs (GemmPlanes)
//   cs  [ngroups][32 rows]                f32 2^s per row
//   cm  [ngroups][32 rows]                f32 offset per row
//
// Quantized activations ([m, k] f32 in, quantize_acts_i8 semantics) are
// written by the quantize kernels in the same row-group form:
//   int8 layout (decode, validation):
//     qa  [mgroups][nb][32 rows][32 B]  int8, MFMA order
//     da  [mgroups][nb][32 rows]        f32 block scale d_a
//     pa  [mgroups][nb][32 rows]        f32 d_a * (float)sum(q_a)  (min term)
//     sa  [mgroups][nb][32 rows]        i32 sum(q_a)
//   f16 layout (encoder GEMM):
//     a16 f16(d_a * q_a * 2^(15 - e_row)) at a16_index (below), one rounding
//     rs  [rows] f32 2^(e_row - 15), applied to the GEMM's output rows
//     ps  [rows] f32 sum over the row's blocks of d_a * sum(q_a)
//
// Decode records (k_gemv, k_gemv_records): per block of an m-row activation,
// the rows' 32 int8 quants in MFMA order, 16 zero bytes (the A operand of
// MFMA lanes whose row is >= m), then 8-entry arrays of -c*sum(q_a), d_a and
// d_a*sum(q_a); see gemv_rec_bytes.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace rw {

constexpr int QK = 32;        // elements per block
constexpr int RG = 32;        // rows per row group
constexpr int OCT = 8;        // blocks per octet

#if defined(__HIPCC__)
#define RW_HD __host__ __device__
#else
#define RW_HD
#endif

RW_HD inline int qs_bytes(int dtype) { return dtype == 8 ? 32 : 16; }
RW_HD inline bool has_min(int dtype) { return dtype == 3 || dtype == 7; }
RW_HD inline bool has_high(int dtype) { return dtype == 6 || dtype == 7; }

// stored position <-> element of a 32-byte MFMA-order block (an involution)
RW_HD inline int mfma_pos(int e) { return (e >= 8 && e < 16) ? e + 8 : (e >= 16 && e < 24) ? e - 8 : e; }

// bit of the permuted high-bit word that holds element e = 4t + u
RW_HD inline int qh_bit(int e) { return (8 * (e & 3) + 4 - (e >> 2)) & 31; }

struct WeightView {
  const uint8_t *qs;
  const uint32_t *qh;
  const uint16_t *d;
  const uint16_t *m;
  int nb, nb_pad, noct, ngroups;
};

// Quantized activations.  The int8 layout (qa, da, pa, sa) serves the
// decode kernels and the validation entries; the GEMM layout (a16, rs) the
// encoder GEMM.  Both index (row group, block, row) by act_slot.
struct ActView {
  const int8_t *qa;     // int8 quants, MFMA order within a block
  const float *da;      // d_a
  const float *pa;      // d_a * sum(q_a)
  const int32_t *sa;    // sum(q_a)
  const uint16_t *a16;  // f16(d_a * q_a * 2^-e_row), GEMM operand order (a16_index)
  const float *rs;      // 2^e_row per row
  const float *ps;      // per row: sum over blocks of d_a * sum(q_a), in f32
  int nb, mgroups;
};

// Weight planes for the encoder GEMM, indexed like qs ([group][nb_pad][32]).
// q8 holds every quant as one byte, in MFMA order within the block, biased to
// unsigned: the 4/5-bit quants as stored (0..15 / 0..31), Q8_0 as q + 128
// (for Q8_0 the plane is qs itself, read with the sign bit flipped).
//
// Each weight row j carries an offset cm[j] (the mean of its finite values
// d*q + m) and a power of two cs[j] = 2^s_j, chosen at upload so that the
// row's largest finite |d*q + m - cm|, |d| or |m - cm| lands in [2^14, 2^15)
// once divided by it.  dm holds f16(d_b / cs[j]) and f16((m_b - cm[j]) /
// cs[j]), so the f16 operand (d*q + m - cm) / cs never overflows, keeps
// f16's full precision for every value above 2^-28 of the row's largest,
// whatever the block scales are, and rounds relative to the row's spread
// rather than to a common offset (a row of Q4_1 / Q5_1 blocks whose mins
// dwarf their ranges).  The GEMM multiplies its output column j by cs[j]
// and adds cm[j] * P_i, P_i the exact sum of activation row i's quantized
// values (ActView::ps), as the reference adds each block's min term
// m_b * d_a * sum(q_a) in f32.
struct GemmPlanes {
  const uint8_t *q8;   // [group][nb_pad][32][32]
  const uint32_t *dm;  // f16 d_b / cs (low half) and (m_b - cm) / cs (high half)
  const float *cs;     // [group * 32] 2^s per weight row (1 for padding rows)
  const float *cm;     // [group * 32] the row's offset (0 for padding rows)
};

// element offsets
RW_HD inline size_t qs_slot(const WeightView &w, int g, int bl, int r) {
  return ((size_t)g * w.nb_pad + bl) * RG + r;
}
RW_HD inline size_t sc_index(const WeightView &w, int g, int bl, int r) {
  return (((size_t)g * w.noct + (bl >> 3)) * RG + r) * OCT + (bl & 7);
}
RW_HD inline size_t act_slot(int nb, int g, int bl, int r) { return ((size_t)g * nb + bl) * RG + r; }

// The f16 activation plane of the encoder GEMM: the 1024 values of (row
// group g, block bl) sit in the order the GEMM's lanes load them,
// [operand p][lane 32h + r][8]: lane (h, r) of the block's p-th MFMA reads
// elements 16p + 8h .. 16p + 8h + 7 of row r as one 16-byte load.
RW_HD inline size_t a16_index(int nb, int g, int bl, int r, int e) {
  return act_slot(nb, g, bl, 0) * QK + (e >> 4) * 512 + (32 * ((e >> 3) & 1) + r) * 8 + (e & 7);
}

}  // namespace rw
