// rw_kernels.hpp -- gfx950 device code for the quantized linear-layer matmul.
//
// Kernels (the arithmetic of src/quant.rs, restated for CDNA4):
//   k_repack        ggml blocks -> resident planes (once per weight)
//   k_dequant       planes -> f32 rows, bit-exact with dequant_row_scalar
//                   (src/quant.rs:528-537)
//   k_quantize      f32 activations -> int8 blocks + d_a + sums, bit-exact
//                   with quantize_acts_i8 (src/quant.rs:691-716)
//   k_quantize_f16  the same quantization, stored as f16 values d_a*q_a
//                   (row-scaled by a power of two) for the encoder GEMM
//   k_block_dots    exact per-block integer sums via int8 MFMA (validation)
//   k_gemm          encoder shape (m > 8): f16 MFMA GEMM of the quantized
//                   activations' values against weights dequantized in
//                   registers (d_b*q_b + m_b, one rounding to f16)
//   k_gemv2         decoder shape (m <= 8): any number of linears in one
//                   launch, activations quantized into LDS, one lane per
//                   weight row, v_dot4_i32_i8 exact block sums
//
// Within a kernel family a row's result never depends on m: every choice
// of order (k splits, chunking) depends on the weight's shape alone.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "rw_layout.hpp"

namespace rw {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------ scalar helpers

// IEEE half -> single with the exact bit rules of model.rs:68-86 (NaN payload
// kept as frac << 13); used where the f32 bits are the product (dequant).
__device__ inline float h2f_exact(uint32_t h) {
  uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1fu, frac = h & 0x3ffu, bits;
  if (exp == 0 && frac == 0) {
    bits = sign << 31;
  } else if (exp == 0) {
    uint32_t p = 31u - (uint32_t)__clz(frac);
    bits = (sign << 31) | ((p + 103u) << 23) | (((frac << (10u - p)) & 0x3ffu) << 13);
  } else if (exp == 0x1f) {
    bits = (sign << 31) | 0x7f800000u | (frac << 13);
  } else {
    bits = (sign << 31) | ((exp + 112u) << 23) | (frac << 13);
  }
  return __uint_as_float(bits);
}

// hardware conversion: identical to h2f_exact for every non-NaN code
__device__ inline float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// Rust `(x).round().clamp(-127.0, 127.0) as i32` (NaN -> 0)
__device__ inline int round_clamp_i8(float v) {
  float r = roundf(v);
  if (r != r) return 0;
  r = r < -127.0f ? -127.0f : r;
  r = r > 127.0f ? 127.0f : r;
  return (int)r;
}

// bytes of a packed-nibble word minus `c` (0 <= byte < 128, c <= byte+128)
__device__ inline uint32_t sub_bytes(uint32_t x, uint32_t c) {
  return ((x | 0x80808080u) - c * 0x01010101u) ^ 0x80808080u;
}

__device__ inline uint32_t rotl(uint32_t x, int t) { return t == 0 ? x : (x << t) | (x >> (32 - t)); }

// --------------------------------------------------------------- k_repack

template <int DT>
__device__ inline void read_block(const uint8_t *p, uint16_t &d, uint16_t &m, uint32_t &qh, uint8_t *q) {
  auto u16 = [&](int o) { return (uint16_t)(p[o] | (p[o + 1] << 8)); };
  auto u32 = [&](int o) {
    return (uint32_t)p[o] | ((uint32_t)p[o + 1] << 8) | ((uint32_t)p[o + 2] << 16) | ((uint32_t)p[o + 3] << 24);
  };
  d = u16(0);
  m = 0;
  qh = 0;
  int qo;
  if (DT == 2) {
    qo = 2;
  } else if (DT == 3) {
    m = u16(2);
    qo = 4;
  } else if (DT == 6) {
    qh = u32(2);
    qo = 6;
  } else if (DT == 7) {
    m = u16(2);
    qh = u32(4);
    qo = 8;
  } else {
    qo = 2;
  }
  const int nq = DT == 8 ? 32 : 16;
  for (int i = 0; i < nq; ++i) q[i] = p[qo + i];
}

// one thread per (row, block) of the padded matrix
template <int DT>
__global__ __launch_bounds__(256) void k_repack(const uint8_t *__restrict__ raw, int n, int nb, uint8_t *qs,
                                                uint32_t *qh, uint16_t *dd, uint16_t *mm, uint32_t *dm,
                                                uint32_t *qhb, int nb_pad, int noct, int ngroups) {
  constexpr int BB = DT == 2 ? 18 : DT == 3 ? 20 : DT == 6 ? 22 : DT == 7 ? 24 : 34;
  constexpr int QSB = DT == 8 ? 32 : 16;
  size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t total = (size_t)ngroups * RG * nb_pad;
  if (t >= total) return;
  int bl = (int)(t % nb_pad);
  int j = (int)(t / nb_pad);
  uint16_t d = 0, m = 0;
  uint32_t h = 0;
  uint8_t q[32];
  for (int i = 0; i < 32; ++i) q[i] = 0;
  if (j < n && bl < nb) read_block<DT>(raw + ((size_t)j * nb + bl) * BB, d, m, h, q);
  WeightView w{nullptr, nullptr, nullptr, nullptr, nb, nb_pad, noct, ngroups};
  int g = j / RG, r = j % RG;
  uint8_t *dst = qs + qs_slot(w, g, bl, r) * QSB;
  if (DT == 8) {
    for (int p = 0; p < 32; ++p) dst[p] = q[mfma_pos(p)];
  } else {
    for (int p = 0; p < 16; ++p) dst[p] = q[p];
  }
  size_t si = sc_index(w, g, bl, r);
  dd[si] = d;
  if (has_min(DT)) mm[si] = m;
  const size_t slot = qs_slot(w, g, bl, r);
  dm[slot] = (uint32_t)d | ((uint32_t)m << 16);
  if (has_high(DT)) {
    uint32_t x = 0;
    for (int e = 0; e < 32; ++e) x |= ((h >> e) & 1u) << qh_bit(e);
    qh[si] = x;
    qhb[slot] = x;
  }
}

// -------------------------------------------------------------- k_dequant

// Element e of block (g, bl, r) as the centered int8 of unpack_block
// (src/quant.rs:98-131).
template <int DT>
__device__ inline int weight_q(const WeightView &w, int g, int bl, int r, int e) {
  if (DT == 8) return (int)(int8_t)w.qs[qs_slot(w, g, bl, r) * 32 + mfma_pos(e)];
  uint8_t byte = w.qs[qs_slot(w, g, bl, r) * 16 + (e & 15)];
  int q = e < 16 ? (byte & 0xf) : (byte >> 4);
  if (has_high(DT)) q |= (int)((w.qh[sc_index(w, g, bl, r)] >> qh_bit(e)) & 1u) << 4;
  if (DT == 2) q -= 8;
  if (DT == 6) q -= 16;
  return q;
}

// one thread per (row, block); x = d*q (exact) + m, one rounding
template <int DT>
__global__ __launch_bounds__(256) void k_dequant(WeightView w, int row0, int nrows, float *__restrict__ out) {
  size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (size_t)nrows * w.nb) return;
  int bl = (int)(t % w.nb);
  int j = row0 + (int)(t / w.nb);
  int g = j / RG, r = j % RG;
  size_t si = sc_index(w, g, bl, r);
  float d = h2f_exact(w.d[si]);
  float m = has_min(DT) ? h2f_exact(w.m[si]) : 0.0f;
  float *o = out + (size_t)(j - row0) * ((size_t)w.nb * QK) + (size_t)bl * QK;
  for (int e = 0; e < QK; ++e) o[e] = __fadd_rn(__fmul_rn(d, (float)weight_q<DT>(w, g, bl, r, e)), m);
}

// ------------------------------------------------------------- k_quantize

// quantize_acts_i8 (src/quant.rs:691-716) for one 32-element block held by
// 8 consecutive lanes, 4 elements each: amax over the block by lane
// shuffles, d = amax / 127 and inv = 1 / d correctly rounded, q = round half
// away from zero of x * inv, clamped to +-127 (NaN -> 0), and sum(q).
struct BlockQuant {
  int q0, q1, q2, q3, sum;
  float d;
};

__device__ inline BlockQuant quantize_block8(float4 x) {
  float amax = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  amax = fmaxf(amax, __shfl_xor(amax, 2));
  amax = fmaxf(amax, __shfl_xor(amax, 4));
  BlockQuant b;
  b.d = __fdiv_rn(amax, 127.0f);
  const float inv = b.d > 0.0f ? __fdiv_rn(1.0f, b.d) : 0.0f;
  b.q0 = round_clamp_i8(__fmul_rn(x.x, inv));
  b.q1 = round_clamp_i8(__fmul_rn(x.y, inv));
  b.q2 = round_clamp_i8(__fmul_rn(x.z, inv));
  b.q3 = round_clamp_i8(__fmul_rn(x.w, inv));
  int s = b.q0 + b.q1 + b.q2 + b.q3;
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  s += __shfl_xor(s, 4);
  b.sum = s;
  return b;
}

__device__ inline uint32_t pack_q4(const BlockQuant &b) {
  return (uint32_t)(b.q0 & 0xff) | ((uint32_t)(b.q1 & 0xff) << 8) | ((uint32_t)(b.q2 & 0xff) << 16) |
         ((uint32_t)(b.q3 & 0xff) << 24);
}

// 8 lanes per (row, block), 4 elements per lane; a wavefront covers 8
// consecutive rows of one row group for one block.  Padded rows (i >= m)
// are written as zeros.
__global__ __launch_bounds__(256) void k_quantize(const float *__restrict__ a, int m, int k, int nb, int mgroups,
                                                  int8_t *__restrict__ qa, float *__restrict__ da,
                                                  float *__restrict__ pa, int32_t *__restrict__ sa) {
  size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t rb = t >> 3;
  int lt = (int)(t & 7);
  if (rb >= (size_t)mgroups * RG * nb) return;  // whole wavefronts exit together
  int r = (int)(rb % RG);
  size_t gb = rb / RG;
  int bl = (int)(gb % nb);
  int g = (int)(gb / nb);
  int i = g * RG + r;
  float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
  if (i < m) x = *reinterpret_cast<const float4 *>(a + (size_t)i * k + (size_t)bl * QK + 4 * lt);
  const BlockQuant bq = quantize_block8(x);
  size_t slot = act_slot(nb, g, bl, r);
  *reinterpret_cast<uint32_t *>(qa + slot * QK + mfma_pos(4 * lt)) = pack_q4(bq);
  if (lt == 0) {
    da[slot] = bq.d;
    pa[slot] = __fmul_rn(bq.d, (float)bq.sum);
    sa[slot] = bq.sum;
  }
}

// Activations for the encoder GEMM, one workgroup per row of the padded
// row groups (rows >= m are written as zeros); 8 lanes per block, 32 blocks
// per pass.  The quantization is quantize_acts_i8's (src/quant.rs:691-716)
// bit for bit; each element is stored as f16(d_a * q_a * 2^-e), in the MFMA
// order of the int8 layout, with e chosen from the row's largest |x| so that
// the largest value lands in [2^14, 2^15): no value overflows, and every
// value keeps f16's full precision unless it is below 2^-28 of the row's
// largest.  rs[row] = 2^e undoes the scaling exactly in the GEMM's epilogue.
// Each row group of the plane is followed by GEMM_PAD_BLOCKS blocks of
// zeros (act_slot16).
__global__ __launch_bounds__(256) void k_quantize_f16(const float *__restrict__ a, int m, int k, int nb,
                                                      uint16_t *__restrict__ a16, float *__restrict__ rs) {
  constexpr int KEEP = 8;  // passes of 32 blocks held in registers (k <= 8192)
  __shared__ float wmax[4];
  const int row = blockIdx.x;
  const int t = threadIdx.x, lb = t >> 3, lt = t & 7;
  const int g = row / RG, r = row % RG;
  // the row's padding blocks (read past the last block by k_gemm): zeros
  for (int bl = nb + lb; bl < nb + GEMM_PAD_BLOCKS; bl += 32)
    *reinterpret_cast<uint2 *>(a16 + act_slot16(nb, g, bl, r) * QK + mfma_pos(4 * lt)) = make_uint2(0u, 0u);
  if (row >= m) {  // uniform per workgroup
    for (int bl = lb; bl < nb; bl += 32)
      *reinterpret_cast<uint2 *>(a16 + act_slot16(nb, g, bl, r) * QK + mfma_pos(4 * lt)) = make_uint2(0u, 0u);
    if (t == 0) rs[row] = 0.0f;
    return;
  }
  const float *x = a + (size_t)row * k;
  float4 xv[KEEP];
  float amax = 0.0f;
#pragma unroll
  for (int p = 0; p < KEEP; ++p) {
    const int bl = 32 * p + lb;
    xv[p] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (bl < nb) xv[p] = *reinterpret_cast<const float4 *>(x + (size_t)bl * QK + 4 * lt);
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(xv[p].x), fabsf(xv[p].y)), fmaxf(fabsf(xv[p].z), fabsf(xv[p].w))));
  }
  for (int bl = 32 * KEEP + lb; bl < nb; bl += 32) {
    const float4 v = *reinterpret_cast<const float4 *>(x + (size_t)bl * QK + 4 * lt);
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((t & 63) == 0) wmax[t >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  int e = 15;  // zero, inf or NaN rows: no scaling
  if (amax > 0.0f && amax <= 3.4028235e38f) {
    frexpf(amax, &e);  // amax in [2^(e-1), 2^e)
    e = max(e, -110);
  }
  const float down = ldexpf(1.0f, 15 - e);
  // whole wavefronts run every pass (the shuffles need all 8 lanes of a
  // block); lanes past the row's blocks quantize zeros and store nothing
  auto emit = [&](float4 v, int bl) __attribute__((always_inline)) {
    const BlockQuant bq = quantize_block8(v);
    if (bl < nb) {
      h2v lo2 = {(_Float16)(__fmul_rn(bq.d, (float)bq.q0) * down), (_Float16)(__fmul_rn(bq.d, (float)bq.q1) * down)};
      h2v hi2 = {(_Float16)(__fmul_rn(bq.d, (float)bq.q2) * down), (_Float16)(__fmul_rn(bq.d, (float)bq.q3) * down)};
      *reinterpret_cast<uint2 *>(a16 + act_slot16(nb, g, bl, r) * QK + mfma_pos(4 * lt)) =
          make_uint2(__builtin_bit_cast(uint32_t, lo2), __builtin_bit_cast(uint32_t, hi2));
    }
  };
#pragma unroll
  for (int p = 0; p < KEEP; ++p)
    if (32 * p < nb) emit(xv[p], 32 * p + lb);
  for (int b0 = 32 * KEEP; b0 < nb; b0 += 32) {
    const int bl = b0 + lb;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (bl < nb) v = *reinterpret_cast<const float4 *>(x + (size_t)bl * QK + 4 * lt);
    emit(v, bl);
  }
  if (t == 0) rs[row] = ldexpf(1.0f, e - 15);
}

// --------------------------------------------------- MFMA operand unpack

// The B operand (weights) of one 32x32x32 MFMA for lane half h and row slot
// r of row group g, block bl; also returns the block's d_b and m_b.
template <int DT>
__device__ inline v4i weight_operand(const WeightView &w, int g, int bl, int r, int h, float &db, float &mb) {
  size_t slot = qs_slot(w, g, bl, r);
  size_t si = sc_index(w, g, bl, r);
  db = h2f(w.d[si]);
  mb = has_min(DT) ? h2f(w.m[si]) : 0.0f;
  if (DT == 8) return *reinterpret_cast<const v4i *>(w.qs + slot * 32 + 16 * h);
  uint2 q = *reinterpret_cast<const uint2 *>(w.qs + slot * 16 + 8 * h);
  uint32_t w0 = q.x & 0x0f0f0f0fu, w1 = q.y & 0x0f0f0f0fu;
  uint32_t w2 = (q.x >> 4) & 0x0f0f0f0fu, w3 = (q.y >> 4) & 0x0f0f0f0fu;
  if (has_high(DT)) {
    uint32_t x = w.qh[si];
    // natural dwords 2h, 2h+1 (elements 8h..8h+7) and 4+2h, 5+2h (16+8h..)
    w0 |= rotl(x, 2 * h) & 0x10101010u;
    w1 |= rotl(x, 2 * h + 1) & 0x10101010u;
    w2 |= rotl(x, 4 + 2 * h) & 0x10101010u;
    w3 |= rotl(x, 5 + 2 * h) & 0x10101010u;
  }
  if (DT == 2) {
    w0 = sub_bytes(w0, 8); w1 = sub_bytes(w1, 8); w2 = sub_bytes(w2, 8); w3 = sub_bytes(w3, 8);
  }
  if (DT == 6) {
    w0 = sub_bytes(w0, 16); w1 = sub_bytes(w1, 16); w2 = sub_bytes(w2, 16); w3 = sub_bytes(w3, 16);
  }
  v4i b;
  b.x = (int)w0; b.y = (int)w1; b.z = (int)w2; b.w = (int)w3;
  return b;
}

// --------------------------------------------------------- k_block_dots

// S[i, j, bl] for every (i < m, j < n); one 32x32 tile per wavefront.
template <int DT>
__global__ __launch_bounds__(64) void k_block_dots(WeightView w, ActView a, int m, int n, int32_t *__restrict__ S) {
  const int l = threadIdx.x, h = l >> 5, r = l & 31;
  const int gn = blockIdx.x, gm = blockIdx.y, bl = blockIdx.z;
  float db, mb;
  v4i bop = weight_operand<DT>(w, gn, bl, r, h, db, mb);
  v4i aop = *reinterpret_cast<const v4i *>(a.qa + act_slot(a.nb, gm, bl, r) * QK + 16 * h);
  v16i zero = {};
  v16i s = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop, zero, 0, 0, 0);
  int j = gn * RG + r;
  for (int v = 0; v < 16; ++v) {
    int i = gm * RG + 8 * (v >> 2) + 4 * h + (v & 3);
    if (i < m && j < n) S[((size_t)i * n + j) * a.nb + bl] = s[v];
  }
}

// ---------------------------------------------------------------- k_gemv2

// Loads and stores through pointers read out of a launch table: the
// compiler cannot tell their address space, and flat accesses also count
// against the LDS wait counter, so every LDS wait would hold for them.
// Address space 1 makes them global_load / global_store (vector-memory
// counter only).  16-byte values go through native vector types, which keep
// the address space where HIP's vector classes do not.
#define RW_GLOBAL_AS __attribute__((address_space(1)))
typedef uint32_t rw_u32x4 __attribute__((ext_vector_type(4)));
typedef float rw_f32x4 __attribute__((ext_vector_type(4)));
__device__ inline uint4 ldg_u4(const void *p) {
  const rw_u32x4 v = *(const rw_u32x4 RW_GLOBAL_AS *)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
typedef uint32_t rw_u32x2 __attribute__((ext_vector_type(2)));
__device__ inline uint2 ldg_u2(const void *p) {
  const rw_u32x2 v = *(const rw_u32x2 RW_GLOBAL_AS *)p;
  return make_uint2(v.x, v.y);
}
__device__ inline float4 ldg_f4(const void *p) {
  const rw_f32x4 v = *(const rw_f32x4 RW_GLOBAL_AS *)p;
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ inline float ldg_f(const void *p) { return *(const float RW_GLOBAL_AS *)p; }
__device__ inline uint32_t ldg_u32(const void *p) { return *(const uint32_t RW_GLOBAL_AS *)p; }
__device__ inline int32_t ldg_i32(const void *p) { return *(const int32_t RW_GLOBAL_AS *)p; }
__device__ inline void stg_f(float *p, float v) { *(float RW_GLOBAL_AS *)(void *)p = v; }

// One linear of a decode-shape launch: out[m, n] = a[m, k] W^T (+ bias).
struct GemvItem {
  WeightView w;
  const float *a;         // f32 activations [m, k] (fused quantization), or
  const int8_t *qa;       // ... an already quantized workspace (act layout)
  const float *qda, *qpa;
  const int32_t *qsa;
  const float *bias;
  float *out;
  int n;
  int wg0;  // first workgroup of this item in the launch
  int lks;  // log2 of the number of wavefronts that split a row's octets
  int pad;
};

// One octet (8 blocks) of one weight row, as loaded: quants, scales, mins and
// (Q5) high-bit words.
template <int DT>
struct OctRegs {
  uint4 q[DT == 8 ? 16 : 8];
  uint4 d, m, h0, h1;
};

template <int DT>
__device__ inline void load_oct(const WeightView &w, int g, int r, int o, OctRegs<DT> &x) {
  const size_t sbase = (((size_t)g * w.noct + o) * RG + r) * OCT;
  x.d = ldg_u4(w.d + sbase);
  if (has_min(DT)) x.m = ldg_u4(w.m + sbase);
  if (has_high(DT)) {
    x.h0 = ldg_u4(w.qh + sbase);
    x.h1 = ldg_u4(w.qh + sbase + 4);
  }
#pragma unroll
  for (int b8 = 0; b8 < OCT; ++b8) {
    const size_t slot = qs_slot(w, g, o * OCT + b8, r);
    if (DT == 8) {
      x.q[2 * b8] = ldg_u4(w.qs + slot * 32);
      x.q[2 * b8 + 1] = ldg_u4(w.qs + slot * 32 + 16);
    } else {
      x.q[b8] = ldg_u4(w.qs + slot * 16);
    }
  }
}

// LDS record of one activation block for the decode kernel: MR x 32 int8
// quants (natural order), MR x {d (f32), c (i32)}, MR x p (f32), padded to
// 16 bytes.  c = -offset * sum(q) seeds the integer dot of the centered
// formats (Q4_0: 8, Q5_0: 16) and is 0 otherwise; p = d * sum(q).
RW_HD constexpr int gemv_rec_bytes(int mr) { return (mr * 44 + 15) & ~15; }

// Decode shape (m = MR <= 8).  One launch covers any number of linears that
// share (dtype, m); workgroup -> item through `wg_item` (GROUPED), or the
// single item `one`.  The activation rows are quantized into LDS with the
// arithmetic of k_quantize (so fused and separate quantization agree bit for
// bit), `ch_oct` octets of blocks at a time, and weight rows stream past them
// one per lane through v_dot4_i32_i8, a whole octet of loads in flight per
// lane (four wavefronts per SIMD hide the latency; a second octet in
// registers would cost one of them).  2^lks of the 4 wavefronts split a
// row's octets (the split depends on the weight only); each walks its blocks
// in increasing order whatever the chunking, and the parts meet in LDS in
// wavefront order: a row's result depends on its weight row and activation
// row alone.  Blocks past nb in the last octet meet zero weight planes (the
// upload writes the padding as zeros) and zero activation records: they add
// exactly +0.
template <int DT, int MR, bool GROUPED>
__global__ __launch_bounds__(256) void k_gemv2(const GemvItem *__restrict__ items, const int *__restrict__ wg_item,
                                               GemvItem one, int ch_oct) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int REC = gemv_rec_bytes(MR), SC = MR * QK, PO = MR * (QK + 8);
  constexpr int OFF = DT == 2 ? 8 : DT == 6 ? 16 : 0;  // centering offset
  // the descriptor is wave-uniform: scalar loads from the table or kernarg
  const GemvItem I = GROUPED ? items[wg_item[blockIdx.x]] : one;
  const WeightView &w = I.w;
  const int nb = w.nb;
  const int lks = I.lks, KS = 1 << lks;
  const int t = threadIdx.x, l = t & 63, wv = t >> 6;
  const int set = wv >> lks, part = wv & (KS - 1);
  const int g_raw = (((int)blockIdx.x - (GROUPED ? I.wg0 : 0)) * (4 >> lks) + set) * 2 + (l >> 5);
  const int g = g_raw < w.ngroups ? g_raw : w.ngroups - 1;
  const int r = l & 31;
  const int o0 = (w.noct * part) >> lks, o1 = (w.noct * (part + 1)) >> lks;

  float acc[MR], accm[MR];
#pragma unroll
  for (int i = 0; i < MR; ++i) {
    acc[i] = 0.0f;
    accm[i] = 0.0f;
  }

  for (int c0 = 0; c0 < w.noct; c0 += ch_oct) {
    const int c1 = min(w.noct, c0 + ch_oct);
    const int bb0 = c0 * OCT, cnb = min(nb, c1 * OCT) - bb0;
    if (c0) __syncthreads();  // every wavefront is done with the previous chunk
    // --- activation records of blocks [bb0, bb0 + cnb) -> LDS; (row, block)
    // pairs in row-major order, 4 passes of 32 per batch so their global
    // loads are in flight together
    const int total = MR * cnb;
    if (I.a) {
      for (int rb0 = 0; rb0 < total; rb0 += 128) {
        float4 x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int rb = rb0 + 32 * u + (t >> 3), lt = t & 7;
          x[u] = make_float4(0.f, 0.f, 0.f, 0.f);
          if (rb < total) {
            const int i = rb / cnb, bl = bb0 + rb % cnb;
            x[u] = ldg_f4(I.a + ((size_t)i * nb + bl) * QK + 4 * lt);
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int rb = rb0 + 32 * u + (t >> 3), lt = t & 7;
          const BlockQuant bq = quantize_block8(x[u]);
          if (rb < total) {
            const int i = rb / cnb, lb = rb % cnb;
            uint8_t *rec = lds + lb * REC;
            *reinterpret_cast<uint32_t *>(rec + i * QK + 4 * lt) = pack_q4(bq);
            if (lt == 0) {
              *reinterpret_cast<int2 *>(rec + SC + 8 * i) = make_int2(__float_as_int(bq.d), -OFF * bq.sum);
              *reinterpret_cast<float *>(rec + PO + 4 * i) = __fmul_rn(bq.d, (float)bq.sum);
            }
          }
        }
      }
    } else {
      // already quantized: row group 0 of the activation layout, MFMA order
      for (int idx = t; idx < total * 8; idx += 256) {
        const int rb = idx >> 3, lt = idx & 7;
        const int i = rb / cnb, lb = rb % cnb;
        const size_t slot = act_slot(nb, 0, bb0 + lb, i);
        uint8_t *rec = lds + lb * REC;
        *reinterpret_cast<uint32_t *>(rec + i * QK + 4 * lt) = ldg_u32(I.qa + slot * QK + mfma_pos(4 * lt));
        if (lt == 0) {
          *reinterpret_cast<int2 *>(rec + SC + 8 * i) =
              make_int2(__float_as_int(ldg_f(I.qda + slot)), -OFF * ldg_i32(I.qsa + slot));
          *reinterpret_cast<float *>(rec + PO + 4 * i) = ldg_f(I.qpa + slot);
        }
      }
    }
    // records of the tail blocks of the last octet: zeros
    const int dead = (c1 - c0) * OCT - cnb;
    for (int z = t; z < dead * (REC / 16); z += 256)
      reinterpret_cast<uint4 *>(lds + cnb * REC)[z] = make_uint4(0, 0, 0, 0);
    __syncthreads();

    // --- weights: one row per lane, this part's octets inside the chunk,
    // each loaded whole (the planes are padded to whole octets)
    const int p0 = max(o0, c0), p1 = min(o1, c1);
    if (p0 < p1) {
      for (int o = p0; o < p1; ++o) {
        OctRegs<DT> cur;
        load_oct<DT>(w, g, r, o, cur);
        const uint32_t dw[4] = {cur.d.x, cur.d.y, cur.d.z, cur.d.w};
        const uint32_t mw[4] = {cur.m.x, cur.m.y, cur.m.z, cur.m.w};
        const uint32_t hw[8] = {cur.h0.x, cur.h0.y, cur.h0.z, cur.h0.w, cur.h1.x, cur.h1.y, cur.h1.z, cur.h1.w};
        const uint8_t *orec = lds + (o - c0) * OCT * REC;
#pragma unroll
        for (int b8 = 0; b8 < OCT; ++b8) {
          const float db = h2f((uint16_t)(dw[b8 >> 1] >> (16 * (b8 & 1))));
          const float mb = has_min(DT) ? h2f((uint16_t)(mw[b8 >> 1] >> (16 * (b8 & 1)))) : 0.0f;
          // the block's 32 quants as 8 natural dwords: dword u = elements 4u..4u+3
          uint32_t wd[8];
          if (DT == 8) {
            // stored in MFMA order: stored dwords 0..7 hold natural dwords 0,1,4,5,2,3,6,7
            const uint4 q0 = cur.q[2 * b8], q1 = cur.q[2 * b8 + 1];
            wd[0] = q0.x; wd[1] = q0.y; wd[4] = q0.z; wd[5] = q0.w;
            wd[2] = q1.x; wd[3] = q1.y; wd[6] = q1.z; wd[7] = q1.w;
          } else {
            const uint4 q = cur.q[b8];
            const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              wd[u] = qq[u] & 0x0f0f0f0fu;
              wd[u + 4] = (qq[u] >> 4) & 0x0f0f0f0fu;
            }
            if (has_high(DT)) {
              const uint32_t x = hw[b8];
#pragma unroll
              for (int u = 0; u < 8; ++u) wd[u] |= rotl(x, u) & 0x10101010u;
            }
          }
          const uint8_t *rec = orec + b8 * REC;
#pragma unroll
          for (int i = 0; i < MR; ++i) {
            const int4 a0 = *reinterpret_cast<const int4 *>(rec + i * QK);
            const int4 a1 = *reinterpret_cast<const int4 *>(rec + i * QK + 16);
            const int2 sc = *reinterpret_cast<const int2 *>(rec + SC + 8 * i);
            // centered formats: sum(q_a*(q-c)) = sum(q_a*q) - c*sum(q_a)
            int s = sc.y;
            s = __builtin_amdgcn_sdot4((int)wd[0], a0.x, s, false);
            s = __builtin_amdgcn_sdot4((int)wd[1], a0.y, s, false);
            s = __builtin_amdgcn_sdot4((int)wd[2], a0.z, s, false);
            s = __builtin_amdgcn_sdot4((int)wd[3], a0.w, s, false);
            s = __builtin_amdgcn_sdot4((int)wd[4], a1.x, s, false);
            s = __builtin_amdgcn_sdot4((int)wd[5], a1.y, s, false);
            s = __builtin_amdgcn_sdot4((int)wd[6], a1.z, s, false);
            s = __builtin_amdgcn_sdot4((int)wd[7], a1.w, s, false);
            acc[i] = __builtin_fmaf(__int_as_float(sc.x) * db, (float)s, acc[i]);
            if (has_min(DT)) accm[i] = __builtin_fmaf(mb, *reinterpret_cast<const float *>(rec + PO + 4 * i), accm[i]);
          }
        }
      }
    }
  }

  float y[MR];
#pragma unroll
  for (int i = 0; i < MR; ++i) y[i] = has_min(DT) ? acc[i] + accm[i] : acc[i];

  const int n = I.n;
  const int col = g_raw * RG + r;
  if (KS == 1) {
    if (g_raw < w.ngroups && col < n)
#pragma unroll
      for (int i = 0; i < MR; ++i) stg_f(I.out + (size_t)i * n + col, I.bias ? y[i] + ldg_f(I.bias + col) : y[i]);
    return;
  }
  __syncthreads();  // the activation LDS is reused for the partial sums
  float *red = reinterpret_cast<float *>(lds);  // [4 wavefronts][MR][64]
#pragma unroll
  for (int i = 0; i < MR; ++i) red[(wv * MR + i) * 64 + l] = y[i];
  __syncthreads();
  if (part == 0 && g_raw < w.ngroups && col < n) {
#pragma unroll
    for (int i = 0; i < MR; ++i) {
      float tt = red[(wv * MR + i) * 64 + l];
      for (int p = 1; p < KS; ++p) tt = tt + red[((wv + p) * MR + i) * 64 + l];
      stg_f(I.out + (size_t)i * n + col, I.bias ? tt + ldg_f(I.bias + col) : tt);
    }
  }
}

// LDS bytes k_gemv2 needs for m rows and chunks of ch_oct octets
RW_HD inline size_t gemv_lds_bytes(int m, int ch_oct) {
  const size_t act = (size_t)ch_oct * OCT * gemv_rec_bytes(m);
  const size_t red = (size_t)4 * m * 64 * 4;
  return act > red ? act : red;
}

// ---------------------------------------------------------------- k_gemm

// Nibble bytes (plus high-bit flags) of one lane's 16 quants -> the two f16
// B operands.  Each byte b becomes the f16 1024 + b (bits 0x6400 | b, one
// v_perm per two of them) and one packed subtract of 1024 + offset leaves the
// exact centered quant.
template <int DT>
__device__ inline void quants_to_f16(const uint32_t (&q)[4], v8h &b0, v8h &b1) {
  constexpr float off = DT == 8 ? 1152.0f : DT == 2 ? 1032.0f : DT == 6 ? 1040.0f : 1024.0f;
  const h2v sub = {(_Float16)(-off), (_Float16)(-off)};
  h2v e[8];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    e[2 * t] = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, q[t], 0x04010400u)) + sub;
    e[2 * t + 1] = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, q[t], 0x04030402u)) + sub;
  }
  b0 = (v8h){e[0].x, e[0].y, e[1].x, e[1].y, e[2].x, e[2].y, e[3].x, e[3].y};
  b1 = (v8h){e[4].x, e[4].y, e[5].x, e[5].y, e[6].x, e[6].y, e[7].x, e[7].y};
}

// The B operand of the two f16 MFMAs of one block for lane half h: items
// 0-7 (first MFMA) are elements 8h..8h+7, items 8-15 (second MFMA) elements
// 16+8h..16+8h+7 -- the order of the activation f16 plane.
template <int DT>
__device__ inline void weight_f16_from(int h, uint4 qs, uint32_t qhw, v8h &b0, v8h &b1) {
  uint32_t q[4];
  if (DT == 8) {
    q[0] = qs.x ^ 0x80808080u; q[1] = qs.y ^ 0x80808080u; q[2] = qs.z ^ 0x80808080u; q[3] = qs.w ^ 0x80808080u;
  } else {
    q[0] = qs.x & 0x0f0f0f0fu;
    q[1] = qs.y & 0x0f0f0f0fu;
    q[2] = (qs.x >> 4) & 0x0f0f0f0fu;
    q[3] = (qs.y >> 4) & 0x0f0f0f0fu;
    if (has_high(DT)) {
      q[0] |= rotl(qhw, 2 * h) & 0x10101010u;
      q[1] |= rotl(qhw, 2 * h + 1) & 0x10101010u;
      q[2] |= rotl(qhw, 4 + 2 * h) & 0x10101010u;
      q[3] |= rotl(qhw, 5 + 2 * h) & 0x10101010u;
    }
  }
  quants_to_f16<DT>(q, b0, b1);
}

// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector
// memory operations of this wavefront are outstanding, nothing else
RW_HD constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }

// One direct global -> LDS load of 16 bytes per lane: lane i's 16 bytes at
// `g` land at LDS byte (m0 + 16 i); m0 (an LDS byte address) must be the
// same in every lane.  Issued as inline asm so that the compiler's wait
// counting never holds an LDS read for it: the caller waits (vmcnt_imm) and
// synchronises before the data is read, and waits for all of them before
// reusing LDS.
__device__ inline void dma16(const void *g, uint32_t m0) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(m0) : "memory");
}
__device__ inline uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}


// Stage layout of k_gemm.  A stage holds KW blocks, one per k-wave, as
// 16-byte chunks; per k-wave: TM activation row groups of f16 values (32
// rows x 4 chunks; chunk c of row r sits at position 4r + (c ^ ((r >> 1) &
// 3)) so the wavefront's 16-byte operand reads cover every LDS bank), then
// 2*TN weight row groups x {quants, high-bit words (Q5), (d, m) pairs}.
// Each piece is a contiguous run of a device plane, so chunk p of a stage
// always comes from one plane offset plus (block index) x (that plane's
// block stride).  A stage moves by direct global -> LDS loads of 64 chunks
// (1 KB) per instruction, UPW per wavefront, padded with loads into an
// unread tail.
template <int DT, int TM, int TN, int KW_>
struct GL {
  static constexpr int KW = KW_, WAVES = 2 * KW_;  // 2 n-waves x KW k-waves
  static constexpr int R = 3;                      // LDS ring buffers
  static constexpr int QSB = DT == 8 ? 32 : 16;   // quant bytes per row-block
  static constexpr bool HH = DT == 6 || DT == 7;
  static constexpr int A_CH = RG * 4;             // chunks per activation row group
  static constexpr int B_QSCH = RG * QSB / 16, B_QHCH = HH ? 8 : 0, B_DMCH = 8;
  static constexpr int B_CH = B_QSCH + B_QHCH + B_DMCH;
  static constexpr int KWC = TM * A_CH + 2 * TN * B_CH;  // chunks per k-wave
  static constexpr int NCH = KW * KWC;                   // chunks per stage
  static constexpr int UPW = (NCH + 64 * WAVES - 1) / (64 * WAVES);
  static constexpr int STAGE = UPW * WAVES * 1024;       // bytes per stage buffer
  static constexpr int A_OFF = 0, B_OFF = TM * A_CH * 16, B_BYTES = B_CH * 16;
  static constexpr int B_QH = B_QSCH * 16, B_DM = (B_QSCH + B_QHCH) * 16;
  static constexpr int PART = TM * TN * 16 * 64 * 4;     // one wavefront's partial sums
  static constexpr int RED = KW > 1 ? 2 * PART : 0;      // k-wave reduction slots
  static constexpr int LDS = R * STAGE > RED ? R * STAGE : RED;
};

// Encoder-shape GEMM (m > 8): out = rs * (A' W'^T) (+ bias), with A' the f16
// values of the quantized activations (k_quantize_f16) and W' = f16(d_b*q_b
// + m_b) formed in registers with one packed f16 fma per two weights (a
// single rounding).  Products of f16 operands are exact and accumulate in
// f32 inside v_mfma_f32_32x32x16_f16, so |y - exact| <= 2^-10 sum|a||w|
// plus the f32 accumulation error.
// A workgroup is 2*KW wavefronts: 2 along n x KW along k (block bl goes to
// k-wave bl % KW); a wavefront owns TM x TN tiles of 32 x 32, the workgroup
// tile is 32*TM activation rows x 64*TN weight rows.  Stages stream through
// a ring of 3 LDS buffers by direct global -> LDS loads, two stages ahead:
// at stage s a wavefront waits for its own loads of stage s, the barrier
// makes the whole stage visible (and frees the buffer of stage s-1), it
// reads its operands, issues stage s+2 and computes.  Each lane's load
// addresses advance by a fixed stride per stage, which runs up to 5*KW
// blocks past a row group's last block: into the activation plane's zeroed
// per-group padding and the weight planes' tail padding (or the next
// weight group), where the block gets zero (d, m), so it adds +0.  The k-waves'
// partials are summed from the last k-wave down (((p3 + p2) + p1) + p0);
// the configuration and the order depend on the weight alone, so a row's
// result never depends on m.
template <int DT, int TM, int TN, int KW>
__global__ __launch_bounds__(128 * KW, 2) void k_gemm(WeightView w, GemmPlanes gp, ActView a, int m, int n,
                                                      const float *__restrict__ bias, float *__restrict__ out) {
  using L = GL<DT, TM, TN, KW>;
  static_assert(5 * KW <= GEMM_PAD_BLOCKS, "loads past the last block stay in the padding");
  constexpr int UPW = L::UPW, R = L::R;
  __shared__ __align__(1024) uint8_t lds[L::LDS];
  const int t = threadIdx.x, l = t & 63, wv = t >> 6;
  const int h = l >> 5, r = l & 31;
  const int nw = wv & 1, kw = wv >> 1;
  int bx, by;
  {
    // XCD-aware order: consecutive workgroup ids go to different XCDs (id % 8);
    // each XCD gets one contiguous band of the row-major tile order, so its
    // L2 holds one band of activation rows.
    const int nx = gridDim.x, total = nx * gridDim.y;
    const int id = blockIdx.y * nx + blockIdx.x;
    const int per = total / 8, rem = total % 8, xcd = id % 8, slot = id / 8;
    const int lin = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
    bx = lin % nx;
    by = lin / nx;
  }
  const int nb = w.nb, ns = (nb + KW - 1) / KW;

  // copy plan: this lane fills stage chunk p = (wv + WAVES u) * 64 + l; its
  // source for stage s is ptr[u] + s * step[u] (block KW s + its k-wave);
  // chunks past the stage re-read the first activation chunk into the
  // unread tail
  const uint8_t *ptr[UPW];
  uint32_t stp[UPW];
#pragma unroll
  for (int u = 0; u < UPW; ++u) {
    const int p = (wv + L::WAVES * u) * 64 + l;
    const int pc = p < L::NCH ? p : 0;
    const int kwc = pc / L::KWC;
    const int cc = pc % L::KWC;
    int stride;
    if (cc < TM * L::A_CH) {
      const int i = cc / L::A_CH, q = cc % L::A_CH;
      const int row = q >> 2, c = (q & 3) ^ ((row >> 1) & 3);
      const int g = min(by * TM + i, a.mgroups - 1);
      ptr[u] = reinterpret_cast<const uint8_t *>(a.a16 + act_slot16(a.nb, g, 0, 0) * QK) + row * 64 + c * 16;
      stride = RG * QK * 2;
    } else {
      const int cb = cc - TM * L::A_CH;
      const int j = cb / L::B_CH, q = cb % L::B_CH;
      const int g = min(bx * 2 * TN + j, w.ngroups - 1);
      const size_t s0 = qs_slot(w, g, 0, 0);
      if (q < L::B_QSCH) {
        ptr[u] = w.qs + s0 * L::QSB + 16 * q;
        stride = RG * L::QSB;
      } else if (q < L::B_QSCH + L::B_QHCH) {
        ptr[u] = reinterpret_cast<const uint8_t *>(gp.qhb + s0) + 16 * (q - L::B_QSCH);
        stride = RG * 4;
      } else {
        ptr[u] = reinterpret_cast<const uint8_t *>(gp.dm + s0) + 16 * (q - L::B_QSCH - L::B_QHCH);
        stride = RG * 4;
      }
    }
    if (p >= L::NCH) stride = 0;
    ptr[u] += (size_t)kwc * stride;
    stp[u] = (uint32_t)(KW * stride);
  }
  // LDS destinations of this wavefront's loads, per ring buffer (uniform)
  uint32_t m0[R][UPW];
#pragma unroll
  for (int q = 0; q < R; ++q)
#pragma unroll
    for (int u = 0; u < UPW; ++u)
      m0[q][u] = __builtin_amdgcn_readfirstlane(lds_addr(lds + q * L::STAGE + (wv + L::WAVES * u) * 1024));
  auto issue = [&](int q) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < UPW; ++u) {
      dma16(ptr[u], m0[q][u]);
      ptr[u] += stp[u];
    }
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (v16f){};
  // epilogue inputs (row scales, bias), loaded now so their latency hides
  // under the k loop; rows and columns past the end read the last one
  float sc[TM][16], bv[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v)
      sc[i][v] = a.rs[min(by * TM + i, a.mgroups - 1) * RG + 8 * (v >> 2) + 4 * h + (v & 3)];
#pragma unroll
  for (int j = 0; j < TN; ++j) bv[j] = bias ? bias[min(((bx * 2 + nw) * TN + j) * RG + r, n - 1)] : 0.0f;

  // the A operand chunk positions of this lane (row r, chunks 2h, 2h+1)
  const int sw = (r >> 1) & 3;
  const int a_off0 = (4 * r + ((2 * h) ^ sw)) * 16, a_off1 = (4 * r + ((2 * h + 1) ^ sw)) * 16;
  // stage s lives in buffer s % 3; the stage count is padded to a multiple
  // of 3 with stages whose blocks are all past nb ((d, m) = 0: they add +0).
  // A step reads all of its operands from LDS before it issues stage s+2.
  auto step = [&](int q, int s) __attribute__((always_inline)) {
    // own loads of stage s done, then everyone's (and stage s-1 read by all);
    // the empty asm statements keep every LDS access on its side of the
    // barrier
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(UPW));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const uint8_t *kb = lds + q * L::STAGE + kw * L::KWC * 16;
    const bool valid = KW * s + kw < nb;
    v8h alo[TM], ahi[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const uint8_t *ag = kb + L::A_OFF + i * L::A_CH * 16;
      alo[i] = *reinterpret_cast<const v8h *>(ag + a_off0);
      ahi[i] = *reinterpret_cast<const v8h *>(ag + a_off1);
    }
    uint4 qw[TN];
    uint32_t qhw[TN], dmw[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const uint8_t *bg = kb + L::B_OFF + (TN * nw + j) * L::B_BYTES;
      if (DT == 8) {
        qw[j] = *reinterpret_cast<const uint4 *>(bg + r * 32 + 16 * h);
      } else {
        const uint2 v = *reinterpret_cast<const uint2 *>(bg + r * 16 + 8 * h);
        qw[j] = make_uint4(v.x, v.y, 0u, 0u);
      }
      qhw[j] = L::HH ? *reinterpret_cast<const uint32_t *>(bg + L::B_QH + 4 * r) : 0u;
      dmw[j] = *reinterpret_cast<const uint32_t *>(bg + L::B_DM + 4 * r);
    }
    __builtin_amdgcn_sched_barrier(0);
    issue((q + 2) % R);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      v8h q0, q1;
      weight_f16_from<DT>(h, qw[j], qhw[j], q0, q1);
      const h2v dmh = __builtin_bit_cast(h2v, valid ? dmw[j] : 0u);
      const v8h dv = dmh.x, mv = dmh.y;
      const v8h wb0 = __builtin_elementwise_fma(q0, dv, mv);
      const v8h wb1 = __builtin_elementwise_fma(q1, dv, mv);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(alo[i], wb0, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi[i], wb1, acc[i][j], 0, 0, 0);
      }
    }
  };
  issue(0);
  issue(1);
  const int nsr = (ns + R - 1) / R * R;
  for (int s = 0; s < nsr; s += R) {
    step(0, s);
    step(1, s + 1);
    step(2, s + 2);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // the last (unused) stages' loads
  __syncthreads();

  // partials from the last k-wave down, through LDS slots [n-wave] of PART
  // bytes
  float *red = reinterpret_cast<float *>(lds + nw * L::PART);
  auto put = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) red[((i * TN + j) * 16 + v) * 64 + l] = acc[i][j][v];
  };
  auto add = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = red[((i * TN + j) * 16 + v) * 64 + l] + acc[i][j][v];
  };
#pragma unroll
  for (int kk = KW - 1; kk > 0; --kk) {
    if (kw == kk) {
      if (kk < KW - 1) add();
      put();
    }
    __syncthreads();
  }
  if (kw != 0) return;
  if (KW > 1) add();

#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int tg = by * TM + i;
    if (tg >= a.mgroups) break;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int cg = (bx * 2 + nw) * TN + j;
      if (cg >= w.ngroups) continue;
      const int col = cg * RG + r;
      if (col >= n) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = tg * RG + 8 * (v >> 2) + 4 * h + (v & 3);
        if (row >= m) continue;
        const float y = acc[i][j][v] * sc[i][v];
        out[(size_t)row * n + col] = bias ? y + bv[j] : y;
      }
    }
  }
}

}  // namespace rw
