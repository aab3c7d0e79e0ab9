// rw_kernels.hpp -- gfx950 device code for the quantized linear-layer matmul.
//
// Kernels (the arithmetic of src/quant.rs, restated for CDNA4):
//   k_repack        ggml blocks -> resident planes (once per weight)
//   k_dequant       planes -> f32 rows, bit-exact with dequant_row_scalar
//   k_matmul_t_f32  the dense f32 tier (tensor::matmul_t), bit-exact
//                   (src/quant.rs:528-537)
//   k_quantize      f32 activations -> int8 blocks + d_a + sums, bit-exact
//                   with quantize_acts_i8 (src/quant.rs:691-716)
//   k_quantize_f16  the same quantization, stored as f16 values d_a*q_a
//                   (row-scaled by a power of two) for the encoder GEMM
//   k_block_dots    exact per-block integer sums via int8 MFMA (validation)
//   k_gemm          encoder shape (m > 8): f16 MFMA GEMM of the quantized
//                   activations' values against weights dequantized in
//                   registers (d_b*q_b + m_b, one rounding to f16)
//   k_gemv          decoder shape (m <= 8): any number of linears in one
//                   launch, activations quantized into LDS, exact block
//                   sums of 32 weight rows x all activation rows per
//                   v_mfma_i32_32x32x32_i8
//
// Within a kernel family a row's result never depends on m: every choice
// of order (k splits, chunking) depends on the weight's shape alone.
#pragma once
#include <hip/hip_fp16.h>
#include <utility>
#include <hip/hip_runtime.h>

#include "rw_layout.hpp"

namespace rw {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));

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
__device__ inline void stg_u32(void *p, uint32_t v) { *(uint32_t RW_GLOBAL_AS *)p = v; }
__device__ inline void stg_u4(void *p, uint4 v) {
  *(rw_u32x4 RW_GLOBAL_AS *)p = rw_u32x4{v.x, v.y, v.z, v.w};
}

// A buffer resource over `bytes` bytes at `base` (gfx9 raw buffer: offsets
// in bytes, loads past the end return zeros)
__device__ inline __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ inline uint4 ldb_u4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ inline uint2 ldb_u2(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
  return make_uint2(v[0], v[1]);
}
// Streaming (read-once) loads: the nt cache policy, so data touched once
// does not displace what the caches should keep
__device__ inline uint4 ldb_u4_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ inline uint2 ldb_u2_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 2);
  return make_uint2(v[0], v[1]);
}
__device__ inline uint32_t ldb_u32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

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

// Rust `(x).round().clamp(-127.0, 127.0) as i32` (NaN -> 0).  In f32
// round-to-nearest arithmetic, x + copysign(0.49999997, x) truncated toward
// zero is round-half-away-from-zero(x) for every f32 x (checked over all
// 2^32 inputs; 0.49999997 rather than 0.5 keeps x = 0.49999997 from
// rounding up to 1).  v_cvt_i32_f32 truncates, saturates +-inf and maps NaN
// to 0; v_med3_i32 clamps.
__device__ inline int round_clamp_i8(float v) {
  const float y = __fadd_rn(v, __builtin_copysignf(0.49999997f, v));
  int r;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(y));
  return min(127, max(-127, r));
}

// bytes of a packed-nibble word minus `c` (0 <= byte < 128, c <= byte+128)
__device__ inline uint32_t sub_bytes(uint32_t x, uint32_t c) {
  return ((x | 0x80808080u) - c * 0x01010101u) ^ 0x80808080u;
}

__device__ inline uint32_t rotl(uint32_t x, int t) { return t == 0 ? x : (x << t) | (x >> (32 - t)); }

// Cross-lane moves within 8-lane groups on the VALU (DPP, gfx9 dpp_ctrl
// encodings) instead of LDS-pipe shuffles
template <int CTRL>
__device__ inline float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// The maximum over each 8-lane group of values that are >= +0 and not NaN,
// in every lane of it.  Such floats order as their bit patterns do, so the
// maxima are integer DPP maxima (no NaN quieting around each move).
__device__ inline float max8_nn(float b) {
  int v = __float_as_int(b);
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false));   // quad_perm [1,0,3,2]: lane i ^ 1
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false));   // quad_perm [2,3,0,1]: lane i ^ 2
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false));  // row_half_mirror: lane 7 - i
  return __int_as_float(v);
}
// max(0, |x|, |y|, |z|, |w|), NaN skipped: the amax fold of
// quantize_acts_i8, which starts at 0 (src/quant.rs:701), over one lane's four
// values (a block's eight lanes then meet in max8_nn)
__device__ inline float amax4(float4 x) {
  return fmaxf(fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))), 0.0f);
}
__device__ inline float max_nn(float a, float b) { return __int_as_float(max(__float_as_int(a), __float_as_int(b))); }
// the sum over each 8-lane group, in every lane of it
__device__ inline int sum8(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false);
  return v;
}
// lane T's value of each 8-lane group, in every lane of it: ds_swizzle in
// bit-mask mode (lane i reads lane (i & 0x18) | T of its 32), one instruction
// on the LDS pipe instead of DPP moves and a select on the VALU
template <int T>
__device__ inline float bcast8(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x18 | (T << 5)));
}

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

// element e of a block read by read_block as the centered int8 of
// unpack_block (src/quant.rs:98-131)
template <int DT>
__device__ inline int raw_q(const uint8_t *q, uint32_t qh, int e) {
  if (DT == 8) return (int)(int8_t)q[e];
  int v = e < 16 ? (q[e] & 15) : (q[e - 16] >> 4);
  if (has_high(DT)) v |= (int)((qh >> e) & 1u) << 4;
  if (DT == 2) v -= 8;
  if (DT == 6) v -= 16;
  return v;
}

__device__ inline float finite_max(float b, float v) {
  const float a = fabsf(v);
  return a <= 3.4028235e38f ? fmaxf(b, a) : b;  // inf and NaN do not count
}

// The GEMM's offset and power-of-two scale of each weight row (GemmPlanes::
// cm, cs): one wavefront per row of the padded matrix, lanes striding over
// the blocks.  cm = the mean of the row's finite values d*q + m (f32, summed
// per lane, then in a butterfly over the lanes) where that mean exceeds the
// values' standard deviation, else 0; the row's largest finite
// |d*q + m - cm|, |d| or |m - cm| is in [2^(E-1), 2^E), and cs = 2^(E-15)
// moves it to [2^14, 2^15).  Finite f16 scales bound E to [-23, 25], so cs is
// a normal f32.  Zero rows (and padding rows) keep cs = 1, cm = 0.
template <int DT>
__global__ __launch_bounds__(256) void k_row_scale(const uint8_t *__restrict__ raw, int n, int nb, int rows,
                                                   float *__restrict__ cs, float *__restrict__ cm) {
  constexpr int BB = DT == 2 ? 18 : DT == 3 ? 20 : DT == 6 ? 22 : DT == 7 ? 24 : 34;
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (j >= rows) return;  // whole wavefronts
  auto fold = [&](float v) __attribute__((always_inline)) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
    return v;
  };
  float sum = 0.0f, cnt = 0.0f;
  if (j < n) {
    for (int bl = lane; bl < nb; bl += 64) {
      uint16_t d, m;
      uint32_t h;
      uint8_t q[32];
      read_block<DT>(raw + ((size_t)j * nb + bl) * BB, d, m, h, q);
      const float df = h2f_exact(d), mf = has_min(DT) ? h2f_exact(m) : 0.0f;
      for (int e = 0; e < QK; ++e) {
        const float v = __fadd_rn(__fmul_rn(df, (float)raw_q<DT>(q, h, e)), mf);
        if (fabsf(v) <= 3.4028235e38f) {
          sum += v;
          cnt += 1.0f;
        }
      }
    }
  }
  sum = fold(sum);
  cnt = fold(cnt);
  const float mean = cnt > 0.0f ? sum / cnt : 0.0f;
  float dev = 0.0f;  // sum of squared deviations from the mean
  if (j < n) {
    for (int bl = lane; bl < nb; bl += 64) {
      uint16_t d, m;
      uint32_t h;
      uint8_t q[32];
      read_block<DT>(raw + ((size_t)j * nb + bl) * BB, d, m, h, q);
      const float df = h2f_exact(d), mf = has_min(DT) ? h2f_exact(m) : 0.0f;
      for (int e = 0; e < QK; ++e) {
        const float v = __fadd_rn(__fmul_rn(df, (float)raw_q<DT>(q, h, e)), mf);
        if (fabsf(v) <= 3.4028235e38f) dev += (v - mean) * (v - mean);
      }
    }
  }
  dev = fold(dev);
  // an offset only where it dominates the spread; elsewhere rounding
  // relative to each value is as good
  const float c = (cnt > 0.0f && mean * mean > dev / cnt) ? mean : 0.0f;
  float mx = 0.0f;
  if (j < n) {
    for (int bl = lane; bl < nb; bl += 64) {
      uint16_t d, m;
      uint32_t h;
      uint8_t q[32];
      read_block<DT>(raw + ((size_t)j * nb + bl) * BB, d, m, h, q);
      const float df = h2f_exact(d), mf = (has_min(DT) ? h2f_exact(m) : 0.0f) - c;
      mx = finite_max(finite_max(mx, df), mf);
      for (int e = 0; e < QK; ++e) mx = finite_max(mx, __fadd_rn(__fmul_rn(df, (float)raw_q<DT>(q, h, e)), mf));
    }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) {
    float sc = 1.0f;
    if (mx > 0.0f) {
      int e;
      frexpf(mx, &e);
      sc = ldexpf(1.0f, e - 15);
    }
    stg_f(cs + j, sc);
    stg_f(cm + j, c);
  }
}

// one thread per (row, block) of the padded matrix; cs and cm from k_row_scale
template <int DT>
__global__ __launch_bounds__(256) void k_repack(const uint8_t *__restrict__ raw, int n, int nb, uint8_t *qs,
                                                uint32_t *qh, uint16_t *dd, uint16_t *mm, uint32_t *dm,
                                                uint8_t *q8, int nb_pad, int noct, int ngroups,
                                                const float *__restrict__ cs, const float *__restrict__ cm) {
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
  const size_t slot = qs_slot(w, g, bl, r);
  uint8_t *dst = qs + slot * QSB;
  if (DT == 8) {
    for (int p = 0; p < 32; ++p) dst[p] = q[mfma_pos(p)];
  } else {
    for (int p = 0; p < 16; ++p) dst[p] = q[p];
    // the GEMM's byte plane: element e = low nibble of byte e (e < 16) or
    // high nibble of byte e - 16, plus its fifth bit for Q5
    uint8_t *d8 = q8 + slot * 32;
    for (int p = 0; p < 32; ++p) {
      const int e = mfma_pos(p);
      uint32_t v = (q[e & 15] >> (4 * (e >> 4))) & 15u;
      if (has_high(DT)) v |= ((h >> e) & 1u) << 4;
      d8[p] = (uint8_t)v;
    }
  }
  size_t si = sc_index(w, g, bl, r);
  dd[si] = d;
  if (has_min(DT)) mm[si] = m;
  // the GEMM's scalars: d and m - cm divided by the row's power of two (one
  // rounding each; inf and NaN stay non-finite).  Blocks past nb are zeros.
  const float inv = __fdiv_rn(1.0f, cs[j]);
  const float mc = bl < nb ? __fsub_rn(has_min(DT) ? h2f_exact(m) : 0.0f, cm[j]) : 0.0f;
  const uint32_t ds = __half_as_ushort(__float2half_rn(__fmul_rn(h2f_exact(d), inv)));
  const uint32_t ms = __half_as_ushort(__float2half_rn(__fmul_rn(mc, inv)));
  dm[slot] = ds | (ms << 16);
  if (has_high(DT)) {
    uint32_t x = 0;
    for (int e = 0; e < 32; ++e) x |= ((h >> e) & 1u) << qh_bit(e);
    qh[si] = x;
  }
}

// ---------------------------------------------------------- k_matmul_t_f32

// The dense f32 tier, C[m, n] = A[m, k] B[n, k]^T (+ bias), with every
// element formed exactly as tensor::dot does (src/tensor.rs:104-129; dot4 at
// 132-158 is the same per row): 8 lane accumulators from +0, acc[l] =
// acc[l] + a[p+l]*b[p+l] with the product and the sum rounded separately,
// over p < k8 = k - k % 8; the tail k8..k summed from -0.0; the lanes summed
// from -0.0 in order, plus the tail; then + bias[j] (add_bias,
// src/tensor.rs:262-272).  So results are bit-identical to the reference's.
// A workgroup computes a 32 x 32 tile from 32-wide k slices of A and B staged
// in LDS; each thread owns 2 x 2 outputs.
__global__ __launch_bounds__(256) void k_matmul_t_f32(const float *__restrict__ a, const float *__restrict__ b,
                                                      const float *__restrict__ bias, float *__restrict__ c,
                                                      int m, int n, int k) {
  __shared__ float As[32][33], Bs[32][33];
  const int t = threadIdx.x, tx = t & 15, ty = t >> 4;
  const int i0 = blockIdx.y * 32, j0 = blockIdx.x * 32;
  const int k8 = k - k % 8;
  float acc[2][2][8];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int v = 0; v < 2; ++v)
#pragma unroll
      for (int l = 0; l < 8; ++l) acc[u][v][l] = 0.0f;
  for (int p0 = 0; p0 < k8; p0 += 32) {
    // 4 values per thread per tile; past k8 (or past m, n) they are +0, whose
    // products (+0) leave every accumulator as it is
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = t + 256 * e, r = idx >> 5, q = idx & 31, p = p0 + q;
      As[r][q] = (i0 + r < m && p < k8) ? a[(size_t)(i0 + r) * k + p] : 0.0f;
      Bs[r][q] = (j0 + r < n && p < k8) ? b[(size_t)(j0 + r) * k + p] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int q0 = 0; q0 < 32; q0 += 8)
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        const float a0 = As[2 * ty][q0 + l], a1 = As[2 * ty + 1][q0 + l];
        const float b0 = Bs[2 * tx][q0 + l], b1 = Bs[2 * tx + 1][q0 + l];
        acc[0][0][l] = __fadd_rn(acc[0][0][l], __fmul_rn(a0, b0));
        acc[0][1][l] = __fadd_rn(acc[0][1][l], __fmul_rn(a0, b1));
        acc[1][0][l] = __fadd_rn(acc[1][0][l], __fmul_rn(a1, b0));
        acc[1][1][l] = __fadd_rn(acc[1][1][l], __fmul_rn(a1, b1));
      }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int i = i0 + 2 * ty + u, j = j0 + 2 * tx + v;
      if (i < m && j < n) {
        float tail = -0.0f;
        for (int p = k8; p < k; ++p) tail = __fadd_rn(tail, __fmul_rn(a[(size_t)i * k + p], b[(size_t)j * k + p]));
        float s = -0.0f;
#pragma unroll
        for (int l = 0; l < 8; ++l) s = __fadd_rn(s, acc[u][v][l]);
        s = __fadd_rn(s, tail);
        if (bias) s = __fadd_rn(s, bias[j]);
        c[(size_t)i * n + j] = s;
      }
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

// gelu(t) = 0.5 t (1 + tanh(z)), z = 0.7978846 (t + 0.044715 t^3) (the tanh
// form of src/tensor.rs:289-305, z in its order), evaluated as
// t / (1 + e^(-2z)): the same function, since 0.5 (1 + tanh z) =
// 1 / (1 + e^(-2z)), on the hardware's exp2 and reciprocal (a few f32
// roundings from the exact value; the tanh form loses more than that to
// cancellation in 1 + tanh z for negative t).  Large negative t gives -0,
// large positive t gives t, -inf gives NaN, as the tanh form does.
__device__ inline float gelu(float t) {
  const float z = 0.7978846f * (t + 0.044715f * t * t * t);
  const float e = __builtin_amdgcn_exp2f(z * -2.8853900817779268f);  // e^(-2z)
  return t * __builtin_amdgcn_rcpf(1.0f + e);
}

// ------------------------------------------------------------- k_quantize

// quantize_acts_i8 (src/quant.rs:691-716) for one 32-element block held by
// 8 consecutive lanes (aligned to 8), 4 elements each: amax over the block by
// DPP moves, d = amax / 127 and inv = 1 / d correctly rounded, q = round half
// away from zero of x * inv, clamped to +-127 (NaN -> 0), and sum(q).
struct BlockQuant {
  int q0, q1, q2, q3, sum;
  float d;
};

__device__ inline BlockQuant quantize_block8(float4 x) {
  const float amax = max8_nn(amax4(x));
  BlockQuant b;
  b.d = __fdiv_rn(amax, 127.0f);
  const float inv = b.d > 0.0f ? __fdiv_rn(1.0f, b.d) : 0.0f;
  b.q0 = round_clamp_i8(__fmul_rn(x.x, inv));
  b.q1 = round_clamp_i8(__fmul_rn(x.y, inv));
  b.q2 = round_clamp_i8(__fmul_rn(x.z, inv));
  b.q3 = round_clamp_i8(__fmul_rn(x.w, inv));
  b.sum = sum8(b.q0 + b.q1 + b.q2 + b.q3);
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

// Activations for the encoder GEMM: WPR wavefronts per row (4 / WPR rows
// per workgroup; rows >= m of the padded row groups are written as zeros).
// A row's blocks go in passes of 8 (1 KB of f32), pass P to wavefront
// P % WPR, whose lanes 8b + t hold elements 4t..4t+3 of block 8P + b.  The
// quantization is quantize_acts_i8's (src/quant.rs:691-716) bit for bit: the
// block maxima come from 8-lane DPP moves, and the correctly rounded
// d = amax / 127 and inv = 1 / d of a wavefront's pass p are computed once, by
// lane p % 8 of each 8-lane group, and read back by DPP broadcast.  Each
// element is stored as f16(q_a * (d_a * 2^(15-e))) at its a16_index position,
// e chosen from the row's largest |x| (the wavefronts of a row meet in LDS)
// so that the largest value lands in [2^14, 2^15): no value overflows, and
// every value keeps f16's full precision unless it is below 2^-28 of the
// row's largest.  d_a * 2^(15-e) is exact unless it falls below f32's normal
// range, and then every q_a times it is zero in f16 either way.
// rs[row] = 2^(e-15) undoes the scaling in the GEMM's epilogue.  NP passes per
// wavefront stay in registers; a longer row is read twice, once for its
// largest |x| and once to quantize.
//
// With LN, each row is first layer-normalized as src/tensor.rs:274-287 does
// (mean, then the mean of squared deviations, inv = 1 / sqrt(var + 1e-5),
// (x - mean) * inv * w + b; sums over the row in tree order), and the
// normalized row is what gets quantized.  LN rows fit one chunk (the host
// checks).
template <int NP, int WPR, bool LN>
__global__ __launch_bounds__(256) void k_quantize_f16(const float *__restrict__ a, int m, int k, int nb,
                                                      uint16_t *__restrict__ a16, float *__restrict__ rs,
                                                      float *__restrict__ ps, const float *__restrict__ lnw,
                                                      const float *__restrict__ lnb) {
  static_assert(WPR == 1 || WPR == 2 || WPR == 4, "a workgroup holds whole rows");
  __shared__ float part_max[4];
  __shared__ float part_sum[3][4];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // workgroup 8j + x runs on XCD x; the 8 * WPR workgroups of a row group
  // all take the same x, so the group's interleaved f16 lines are written
  // through one L2
  constexpr int WPG = 8 * WPR;  // workgroups per row group
  const int x8 = blockIdx.x & 7, j = blockIdx.x >> 3;
  const int g = 8 * (j / WPG) + x8;
  if (g * RG >= ((m + RG - 1) / RG) * RG) return;  // a slot past the last row group (whole workgroup)
  const int r = (j % WPG) * (4 / WPR) + wv / WPR, part = wv % WPR;
  const int row = g * RG + r;
  const int lb = lane >> 3, lt = lane & 7;
  // stores: the plane as a buffer, this lane's place in a block as the
  // vector offset, the block's place as the scalar offset
  const auto ro = buffer_rsrc(a16, (uint32_t)((size_t)(m + RG - 1) / RG * RG * (size_t)k * 2));
  const uint32_t voff = (uint32_t)(a16_index(nb, g, 0, r, 4 * lt) - a16_index(nb, g, 0, 0, 0)) * 2 +
                        (uint32_t)lb * 2048u;
  const uint32_t gbase = (uint32_t)a16_index(nb, g, 0, 0, 0) * 2;
  const bool live = row < m;  // uniform per row
  const float *x = a + (size_t)row * k;
  constexpr int CB = 8 * NP * WPR;  // blocks per chunk (all wavefronts of the row)
  const int nch = (nb + CB - 1) / CB;
  // first block of this wavefront's pass p in chunk c
  auto first = [&](int c, int p) __attribute__((always_inline)) { return c * CB + 8 * (p * WPR + part); };
  float4 v[NP];
  float bam[NP];
  auto load = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int bl = first(c, p) + lb;
      v[p] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (bl < nb) v[p] = ldg_f4(x + (size_t)bl * QK + 4 * lt);
    }
  };
  auto block_max = [&]() __attribute__((always_inline)) {
    float amax = 0.0f;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      bam[p] = max8_nn(amax4(v[p]));
      amax = max_nn(amax, bam[p]);
    }
    return amax;
  };
  // the row sum over all wavefronts of the row (tree order)
  auto row_sum = [&](float t, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) t += __shfl_xor(t, o);
    if (WPR > 1) {
      if (lane == 0) part_sum[slot][wv] = t;
      __syncthreads();
      t = part_sum[slot][wv - part];
#pragma unroll
      for (int jj = 1; jj < WPR; ++jj) t += part_sum[slot][wv - part + jj];
    }
    return t;
  };
  if constexpr (LN) {
    // every wavefront takes part in both reductions (their barriers)
    float t = 0.0f;
    if (live) {
      load(0);
#pragma unroll
      for (int p = 0; p < NP; ++p) t += (v[p].x + v[p].y) + (v[p].z + v[p].w);
    }
    const float mean = __fdiv_rn(row_sum(t, 0), (float)k);
    t = 0.0f;
    if (live) {
#pragma unroll
      for (int p = 0; p < NP; ++p)
        if (first(0, p) + lb < nb) {
          const float d0 = v[p].x - mean, d1 = v[p].y - mean, d2 = v[p].z - mean, d3 = v[p].w - mean;
          t += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
        }
    }
    const float var = __fdiv_rn(row_sum(t, 1), (float)k);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(var + 1e-5f));
    if (live) {
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int bl = first(0, p) + lb;
        if (bl < nb) {
          const float4 w4 = ldg_f4(lnw + (size_t)bl * QK + 4 * lt), b4 = ldg_f4(lnb + (size_t)bl * QK + 4 * lt);
          v[p].x = (v[p].x - mean) * inv * w4.x + b4.x;
          v[p].y = (v[p].y - mean) * inv * w4.y + b4.y;
          v[p].z = (v[p].z - mean) * inv * w4.z + b4.z;
          v[p].w = (v[p].w - mean) * inv * w4.w + b4.w;
        }
      }
    }
  }
  float amax = 0.0f;  // the block maxima are >= 0 and never NaN: integer maxima
  if (live) {
    for (int c = 0; c < nch; ++c) {
      if (!LN) load(c);
      amax = max_nn(amax, block_max());
    }
    amax = max_nn(amax, __shfl_xor(amax, 8));
    amax = max_nn(amax, __shfl_xor(amax, 16));
    amax = max_nn(amax, __shfl_xor(amax, 32));
  }
  if (WPR > 1) {  // every wavefront reaches the barrier
    if (lane == 0) part_max[wv] = amax;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < WPR; ++j) amax = max_nn(amax, part_max[wv - part + j]);
  }
  if (!live) {
    for (int c = 0; c < nch; ++c)
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int bl = first(c, p) + lb;
        if (bl < nb) *reinterpret_cast<uint2 *>(a16 + a16_index(nb, g, bl, r, 4 * lt)) = make_uint2(0u, 0u);
      }
    row_sum(0.0f, 2);  // the row-sum reduction's barrier, as the live rows
    if (part == 0 && lane == 0) {
      rs[row] = 0.0f;
      ps[row] = 0.0f;
    }
    return;
  }
  int e = 15;  // zero, inf or NaN rows: no scaling
  if (amax > 0.0f && amax <= 3.4028235e38f) {
    frexpf(amax, &e);  // amax in [2^(e-1), 2^e)
    e = max(e, -110);
  }
  const float down = ldexpf(1.0f, 15 - e);
  constexpr int NC = (NP + 7) / 8;
  float ptot = 0.0f;  // this lane's blocks' d_a * sum(q_a) (one lane per block)
  for (int c = 0; c < nch; ++c) {
    if (nch > 1) {
      load(c);
      block_max();
    }
    // lane t of each 8-lane group divides for the passes p = t (mod 8)
    float dv[NC], iv[NC];
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      float b = bam[8 * cc];
#pragma unroll
      for (int t = 1; t < 8; ++t)
        if (8 * cc + t < NP) b = lt == t ? bam[8 * cc + t] : b;
      dv[cc] = __fdiv_rn(b, 127.0f);
      iv[cc] = dv[cc] > 0.0f ? __fdiv_rn(1.0f, dv[cc]) : 0.0f;
    }
    auto pass = [&](auto pc) __attribute__((always_inline)) {
      constexpr int p = decltype(pc)::value;
      const int b0 = first(c, p);
      if (b0 >= nb) return;  // uniform
      const float inv = bcast8<p & 7>(iv[p >> 3]);
      const float da = bcast8<p & 7>(dv[p >> 3]);
      const float dd = da * down;
      const int q0 = round_clamp_i8(__fmul_rn(v[p].x, inv)), q1 = round_clamp_i8(__fmul_rn(v[p].y, inv));
      const int q2 = round_clamp_i8(__fmul_rn(v[p].z, inv)), q3 = round_clamp_i8(__fmul_rn(v[p].w, inv));
      // the block's sum(q_a) (exact integers), times d_a, counted once
      const int bsum = sum8(q0 + q1 + q2 + q3);
      if (lt == 0) ptot += __fmul_rn(da, (float)bsum);
      const h2v lo2 = {(_Float16)__fmul_rn((float)q0, dd), (_Float16)__fmul_rn((float)q1, dd)};
      const h2v hi2 = {(_Float16)__fmul_rn((float)q2, dd), (_Float16)__fmul_rn((float)q3, dd)};
      if (b0 + lb < nb) {
        __builtin_amdgcn_raw_buffer_store_b64(
            (rw_u32x2){__builtin_bit_cast(uint32_t, lo2), __builtin_bit_cast(uint32_t, hi2)}, ro, voff,
            gbase + (uint32_t)b0 * 2048u, 0);
      }
    };
    [&]<int... P>(std::integer_sequence<int, P...>) {
      (pass(std::integral_constant<int, P>{}), ...);
    }(std::make_integer_sequence<int, NP>{});
  }
  ptot = row_sum(ptot, 2);
  if (part == 0 && lane == 0) {
    rs[row] = ldexpf(1.0f, e - 15);
    ps[row] = ptot;
  }
}

// The maximum over each quad of lanes of values that are >= +0 and not NaN
// (integer DPP maxima, as max8_nn)
__device__ inline float max4_nn(float b) {
  int v = __float_as_int(b);
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false));  // quad_perm [1,0,3,2]
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false));  // quad_perm [2,3,0,1]
  return __int_as_float(v);
}
// lane S of each quad's value, in every lane of the quad (DPP quad_perm)
template <int S>
__device__ inline float quad_bcast(float v) {
  constexpr int CTRL = S | (S << 2) | (S << 4) | (S << 6);
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// the value of the lane N above within each row of 16 lanes: DPP row_ror
// by 16 - N (lane i reads lane (i + N) mod 16)
template <int N>
__device__ inline float row_next(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + (16 - N), 0xf, 0xf, false));
}

// k_quantize_f16<NP, WPR, false> with R = 4 or 8 rows per wavefront: the
// same plane, rs and ps, bit for bit, written in runs of R rows.  The plane
// holds a block's 16-byte pieces of the 32 rows of a row group next to each
// other (a16_index), so a lane that owns 8 consecutive elements of one row
// stores 16 bytes, and the R lanes holding the same piece of R consecutive
// rows store R x 16 contiguous bytes; k_quantize_f16's lanes store 8-byte
// pieces of one row, 32 separate pieces per instruction, which costs the L2
// four to eight times the write requests (2 us of the 15 us at
// k = 5120, m = 1500).
// A workgroup holds R rows and WPR x SW wavefronts.  Wavefront w = P SW + s
// takes part P of each row as k_quantize_f16 deals it (blocks
// 8 (p WPR + P) + lb, p < NP) and of those the blocks lb in
// [LB s, LB s + LB), LB = 8 / SW, for all R rows; lane = L rr + 4 jb + q
// (L = 64 / R lanes per row) holds elements 8q..8q+7 of block jb of a pass
// of BP = L / 4 blocks.  The quantization of each element is
// k_quantize_f16's.  The row's ps sums the same per-block terms in the same
// tree: a lane's accumulator u runs over p in order as k_quantize_f16's
// lane does; the pairs (lb, lb ^ 1), then (lb, lb ^ 2), then (lb, lb ^ 4) of
// its shuffle tree are formed here across jb (DPP), across the
// accumulators, or across the wavefronts s (LDS), in the same pairing; the
// parts P are added in order.  Each quad's lanes divide for the passes
// h = q (mod 4) and pass the results by DPP.
template <int R, int NP, int WPR, int SW>
__global__ __launch_bounds__(64 * WPR * SW) void k_quantize_f16_rows(const float *__restrict__ a, int m, int k, int nb,
                                                                     uint16_t *__restrict__ a16, float *__restrict__ rs,
                                                                     float *__restrict__ ps) {
  static_assert(R == 4 || R == 8, "4 or 8 rows per wavefront");
  static_assert(WPR == 2 || WPR == 4, "parts of k_quantize_f16<NP, WPR>");
  constexpr int L = 64 / R, BP = L / 4, NW = WPR * SW, LB = 8 / SW;
  static_assert(SW >= 1 && LB % BP == 0, "a wavefront's blocks of a group are whole passes");
  constexpr int U = LB / BP, H = NP * U, RPG = RG / R;
  __shared__ int smax[NW][R];
  __shared__ float ssum[NW][R];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int P = w / SW, s = w % SW;
  // workgroup 8j + x runs on XCD x; the RPG workgroups of a row group all
  // take the same x, so the group's plane lines are written through one L2
  const int x8 = blockIdx.x & 7, j = blockIdx.x >> 3;
  const int g = 8 * (j / RPG) + x8;
  if (g * RG >= ((m + RG - 1) / RG) * RG) return;  // a slot past the last row group (whole workgroup)
  const int rr = lane / L, jb = (lane % L) >> 2, q = lane & 3;
  const int r = (j % RPG) * R + rr, row = g * RG + r;
  const bool live = row < m;  // rows >= m of the last row group are written as zeros
  const float *x = a + (size_t)row * k;
  // first block of pass h: group p = h / U of part P, blocks lb = LB s + BP (h % U) + jb
  auto blk0 = [&](int h) __attribute__((always_inline)) { return 8 * ((h / U) * WPR + P) + LB * s + BP * (h % U); };
  float4 v[H][2];
#pragma unroll
  for (int h = 0; h < H; ++h) {
    const int bl = blk0(h) + jb;
    v[h][0] = v[h][1] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live && bl < nb) {
      v[h][0] = ldg_f4(x + (size_t)bl * QK + 8 * q);
      v[h][1] = ldg_f4(x + (size_t)bl * QK + 8 * q + 4);
    }
  }
  // block maxima (in every lane of the block's quad) and the row's largest |x|
  float bm[H];
  int amx = 0;
#pragma unroll
  for (int h = 0; h < H; ++h) {
    bm[h] = max4_nn(max_nn(amax4(v[h][0]), amax4(v[h][1])));
    amx = max(amx, __float_as_int(bm[h]));
  }
  if constexpr (L == 16) {
    amx = max(amx, __float_as_int(row_next<4>(__int_as_float(amx))));
    amx = max(amx, __float_as_int(row_next<8>(__int_as_float(amx))));
  } else {
    amx = max(amx, __builtin_amdgcn_update_dpp(0, amx, 0x141, 0xf, 0xf, false));  // row_half_mirror: the other quad
  }
  if (lane % L == 0) smax[w][rr] = amx;
  __syncthreads();
#pragma unroll
  for (int u = 0; u < NW; ++u) amx = max(amx, smax[u][rr]);
  const float amax = __int_as_float(amx);
  int e = 15;  // zero, inf or NaN rows: no scaling
  if (amax > 0.0f && amax <= 3.4028235e38f) {
    frexpf(amax, &e);  // amax in [2^(e-1), 2^e)
    e = max(e, -110);
  }
  const float down = ldexpf(1.0f, 15 - e);
  constexpr int ND = (H + 3) / 4;
  float dv[ND], iv[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) {
    float b = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      if (4 * i + t < H) b = q == t ? bm[4 * i + t] : b;
    dv[i] = __fdiv_rn(b, 127.0f);
    iv[i] = dv[i] > 0.0f ? __fdiv_rn(1.0f, dv[i]) : 0.0f;
  }
  const auto ro = buffer_rsrc(a16, (uint32_t)((size_t)(m + RG - 1) / RG * RG * (size_t)k * 2));
  const uint32_t voff = (uint32_t)(a16_index(nb, 0, jb, r, 8 * q) * 2);
  const uint32_t gbase = (uint32_t)a16_index(nb, g, 0, 0, 0) * 2;
  float acc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) acc[u] = 0.0f;
  auto pass = [&](auto hc) __attribute__((always_inline)) {
    constexpr int h = decltype(hc)::value;
    const int b0 = blk0(h);
    if (b0 >= nb) return;  // uniform
    const float da = quad_bcast<h & 3>(dv[h >> 2]);
    const float inv = quad_bcast<h & 3>(iv[h >> 2]);
    const float dd = da * down;
    const float xs[8] = {v[h][0].x, v[h][0].y, v[h][0].z, v[h][0].w, v[h][1].x, v[h][1].y, v[h][1].z, v[h][1].w};
    int qv[8], sq = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      qv[u] = round_clamp_i8(__fmul_rn(xs[u], inv));
      sq += qv[u];
    }
    // the block's sum(q_a) (exact integers), times d_a
    sq += __builtin_amdgcn_update_dpp(0, sq, 0xB1, 0xf, 0xf, false);
    sq += __builtin_amdgcn_update_dpp(0, sq, 0x4E, 0xf, 0xf, false);
    acc[h % U] += __fmul_rn(da, (float)sq);
    uint32_t wd[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const h2v t2 = {(_Float16)__fmul_rn((float)qv[2 * u], dd), (_Float16)__fmul_rn((float)qv[2 * u + 1], dd)};
      wd[u] = __builtin_bit_cast(uint32_t, t2);
    }
    if (b0 + jb < nb)
      __builtin_amdgcn_raw_buffer_store_b128((rw_u32x4){wd[0], wd[1], wd[2], wd[3]}, ro, voff,
                                             gbase + (uint32_t)b0 * 2048u, 0);
  };
  [&]<int... Hs>(std::integer_sequence<int, Hs...>) {
    (pass(std::integral_constant<int, Hs>{}), ...);
  }(std::make_integer_sequence<int, H>{});
  // ps: pairs across jb (the block 4 lanes above, then 8 above), then
  // across the accumulators, then across the wavefronts s, then the parts
  float xu[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float t = acc[u];
    if constexpr (BP == 4) {
      t = t + row_next<4>(t);
      t = t + row_next<8>(t);
    } else {
      t = t + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), 0x104, 0xf, 0xf, false));  // row_shl:4
    }
    xu[u] = t;
  }
  float y = xu[0];
  if constexpr (U == 2) y = xu[0] + xu[1];
  if constexpr (U == 4) y = (xu[0] + xu[1]) + (xu[2] + xu[3]);
  if (lane % L == 0) ssum[w][rr] = y;
  __syncthreads();
  if (w == 0 && lane % L == 0) {
    auto part_total = [&](int p) __attribute__((always_inline)) {
      const float *t = &ssum[p * SW][0];
      if constexpr (SW == 1) return t[rr];
      else if constexpr (SW == 2) return t[rr] + t[R + rr];
      else return (t[rr] + t[R + rr]) + (t[2 * R + rr] + t[3 * R + rr]);
    };
    float tot = part_total(0);
#pragma unroll
    for (int p = 1; p < WPR; ++p) tot = tot + part_total(p);
    rs[row] = live ? ldexpf(1.0f, e - 15) : 0.0f;
    ps[row] = live ? tot : 0.0f;
  }
}

// The second half of k_quantize_f16 for rows a GEMM_QUANT epilogue has
// already quantized: q (int8, [row group][block][32 rows][32]) and each
// block's largest |y| (am, [row group][block][32 rows]) give the row's
// exponent e (the largest block maximum),
// d_a = amax / 127 per block, and the f16 values q_a * (d_a * 2^(15-e)),
// rs and ps -- every lane, pass and reduction as k_quantize_f16<NP, WPR,
// false> runs them, so the plane is the one k_quantize_f16 writes for the
// f32 rows those quants came from, bit for bit.
template <int NP, int WPR>
__global__ __launch_bounds__(256) void k_quantize_finish(const int8_t *__restrict__ q, const float *__restrict__ am,
                                                         int m, int k, int nb, uint16_t *__restrict__ a16,
                                                         float *__restrict__ rs, float *__restrict__ ps) {
  static_assert(WPR == 1 || WPR == 2 || WPR == 4, "a workgroup holds whole rows");
  __shared__ float part_max[4];
  __shared__ float part_sum[4];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int WPG = 8 * WPR;
  const int x8 = blockIdx.x & 7, j = blockIdx.x >> 3;
  const int g = 8 * (j / WPG) + x8;
  if (g * RG >= ((m + RG - 1) / RG) * RG) return;
  const int r = (j % WPG) * (4 / WPR) + wv / WPR, part = wv % WPR;
  const int row = g * RG + r;
  const int lb = lane >> 3, lt = lane & 7;
  const auto ro = buffer_rsrc(a16, (uint32_t)((size_t)(m + RG - 1) / RG * RG * (size_t)k * 2));
  const uint32_t voff = (uint32_t)(a16_index(nb, g, 0, r, 4 * lt) - a16_index(nb, g, 0, 0, 0)) * 2 +
                        (uint32_t)lb * 2048u;
  const uint32_t gbase = (uint32_t)a16_index(nb, g, 0, 0, 0) * 2;
  const bool live = row < m;
  const int8_t *qr = q + act_slot(nb, g, 0, r) * QK;  // block bl at + bl * RG * QK
  const float *ar = am + act_slot(nb, g, 0, r);        // block bl at + bl * RG
  constexpr int CB = 8 * NP * WPR;
  const int nch = (nb + CB - 1) / CB;
  auto first = [&](int c, int p) __attribute__((always_inline)) { return c * CB + 8 * (p * WPR + part); };
  uint32_t qv[NP];
  float bam[NP];
  auto load = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int bl = first(c, p) + lb;
      qv[p] = 0u;
      bam[p] = 0.0f;
      if (bl < nb) {
        qv[p] = ldg_u32(qr + (size_t)bl * (RG * QK) + 4 * lt);
        bam[p] = ldg_f(ar + (size_t)bl * RG);
      }
    }
  };
  float amax = 0.0f;
  if (live) {
    for (int c = 0; c < nch; ++c) {
      load(c);
#pragma unroll
      for (int p = 0; p < NP; ++p) amax = max_nn(amax, bam[p]);
    }
    amax = max_nn(amax, __shfl_xor(amax, 8));
    amax = max_nn(amax, __shfl_xor(amax, 16));
    amax = max_nn(amax, __shfl_xor(amax, 32));
  }
  if (WPR > 1) {
    if (lane == 0) part_max[wv] = amax;
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < WPR; ++jj) amax = max_nn(amax, part_max[wv - part + jj]);
  }
  auto row_sum = [&](float t) __attribute__((always_inline)) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) t += __shfl_xor(t, o);
    if (WPR > 1) {
      if (lane == 0) part_sum[wv] = t;
      __syncthreads();
      t = part_sum[wv - part];
#pragma unroll
      for (int jj = 1; jj < WPR; ++jj) t += part_sum[wv - part + jj];
    }
    return t;
  };
  if (!live) {
    for (int c = 0; c < nch; ++c)
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int bl = first(c, p) + lb;
        if (bl < nb) *reinterpret_cast<uint2 *>(a16 + a16_index(nb, g, bl, r, 4 * lt)) = make_uint2(0u, 0u);
      }
    row_sum(0.0f);
    if (part == 0 && lane == 0) {
      rs[row] = 0.0f;
      ps[row] = 0.0f;
    }
    return;
  }
  int e = 15;
  if (amax > 0.0f && amax <= 3.4028235e38f) {
    frexpf(amax, &e);
    e = max(e, -110);
  }
  const float down = ldexpf(1.0f, 15 - e);
  float ptot = 0.0f;
  for (int c = 0; c < nch; ++c) {
    if (nch > 1) load(c);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int b0 = first(c, p);
      if (b0 >= nb) continue;  // uniform
      const float da = __fdiv_rn(bam[p], 127.0f);
      const float dd = da * down;
      const int q0 = (int)(int8_t)(qv[p] & 0xff), q1 = (int)(int8_t)((qv[p] >> 8) & 0xff);
      const int q2 = (int)(int8_t)((qv[p] >> 16) & 0xff), q3 = (int)(int8_t)(qv[p] >> 24);
      const int bsum = sum8(q0 + q1 + q2 + q3);
      if (lt == 0) ptot += __fmul_rn(da, (float)bsum);
      const h2v lo2 = {(_Float16)__fmul_rn((float)q0, dd), (_Float16)__fmul_rn((float)q1, dd)};
      const h2v hi2 = {(_Float16)__fmul_rn((float)q2, dd), (_Float16)__fmul_rn((float)q3, dd)};
      if (b0 + lb < nb) {
        __builtin_amdgcn_raw_buffer_store_b64(
            (rw_u32x2){__builtin_bit_cast(uint32_t, lo2), __builtin_bit_cast(uint32_t, hi2)}, ro, voff,
            gbase + (uint32_t)b0 * 2048u, 0);
      }
    }
  }
  ptot = row_sum(ptot);
  if (part == 0 && lane == 0) {
    rs[row] = ldexpf(1.0f, e - 15);
    ps[row] = ptot;
  }
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

// ----------------------------------------------------------------- k_gemv


// One linear of a decode-shape launch: out[m, n] = a[m, k] W^T (+ bias).
struct GemvItem {
  WeightView w;
  const float *a;         // f32 activations [m, k] (fused quantization), or
  const int8_t *qa;       // ... an already quantized workspace (act layout)
  const float *qda, *qpa;
  const int32_t *qsa;
  const float *bias;
  float *out;
  uint8_t *rec;  // activation records [noct*8][gemv_rec_bytes(m)] written by
                 // k_gemv_records (grouped launches), or NULL
  const float *lnw, *lnb;  // single / set launches: layernorm the rows of `a` first (or NULL)
  int n;
  int lks;    // log2 of the number of wavefronts that split a row's octets
  int flags;  // GEMM_GELU, GEMM_ACC: the GEMM's epilogue options; GEMV_REC_OUT
};
// Single and set launches: also write the outputs' activation records to
// `rec` ([n / 32][gemv_rec_bytes(m)], the layout k_gemv_records writes), for
// a next product of the same dtype whose item reads them (a == NULL, rec
// set) instead of quantizing these rows in every workgroup.
constexpr int GEMV_REC_OUT = 8;

// Up to GEMV_SET linears of one dtype that read one activation, launched
// together without a device table: workgroups [end[t-1], end[t]) run item t.
constexpr int GEMV_SET = 4;
constexpr int GEMV_MR_MAX = 8;  // activation rows k_gemv takes
struct GemvSet {
  GemvItem it[GEMV_SET];
  int end[GEMV_SET];
  int count;
};


// LDS record of one activation block for the decode kernel (m = MR rows):
//   [0, 32 MR)         the rows' int8 quants, MFMA order (the A operand)
//   [32 MR, +16)       zeros: the A operand of lanes whose row is >= MR
//   SEED: i32[8]       -c * sum(q_a), c the centering offset of the format
//                      (Q4_0: 8, Q5_0: 16, else 0)
//   DA:   f32[8]       d_a
//   PA:   f32[8]       d_a * sum(q_a) (min term)
// Entries of rows >= MR in the three arrays are zero.
RW_HD constexpr int gemv_rec_bytes(int mr) { return 32 * mr + 16 + 96; }

// Zero the parts of record slots [0, nslots) that gemv_fill never writes:
// the 16-byte zero A operand and the SEED / DA / PA entries of rows >= MR.
template <int MR>
__device__ inline void gemv_zero_slots(uint8_t *lds, int nslots, int t) {
  constexpr int REC = gemv_rec_bytes(MR), ZO = 32 * MR, SO = ZO + 16;
  constexpr int NZ = 8 - MR > 0 ? 8 - MR : 1, ZW = 4 + 3 * (8 - MR);
  for (int z = t; z < nslots * ZW; z += 256) {
    const int s = z / ZW, u = z - s * ZW;
    const int off = u < 4 ? ZO + 4 * u : SO + 32 * ((u - 4) / NZ) + 4 * (MR + (u - 4) % NZ);
    *reinterpret_cast<uint32_t *>(lds + s * REC + off) = 0u;
  }
}

// Activation records of octets [c0, c1) (blocks [8 c0, min(nb, 8 c1))) into
// LDS at `base`: quantized here from f32 (I.a, the arithmetic of k_quantize,
// so fused and separate quantization agree bit for bit)
// or copied from an already quantized workspace (I.qa).  (block, row) pairs
// block-major, U passes of 32 per batch (4, or 8 for one row in the latency
// form: fc2's 160 blocks in one round of loads; 5-row sets measured slower
// with 8) so their global loads are in flight together.  Records of the
// tail blocks past nb are zeroed.
// With I.lnw the rows are layernormed first (mean ln[i] and inverse deviation
// ln[GEMV_MR_MAX + i] of row i, in LDS; then (x - mean) * inv * w + b,
// src/tensor.rs:274-287) and the result quantized.
template <int DT, int MR, int U = 4>
__device__ inline void gemv_fill(const GemvItem &I, int nb, int c0, int c1, uint8_t *base, int t,
                                 const float *ln) {
  constexpr int REC = gemv_rec_bytes(MR), ZO = 32 * MR, SO = ZO + 16, DO = SO + 32, PO = DO + 32;
  constexpr int OFF = DT == 2 ? 8 : DT == 6 ? 16 : 0;
  const int bb0 = c0 * OCT, cnb = min(nb, c1 * OCT) - bb0;
  const int total = MR * cnb;
  if (I.a) {
    // U loads per thread in flight per round (32 U (row, block) pairs)
    for (int rb0 = 0; rb0 < total; rb0 += 32 * U) {
      float4 x[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int rb = rb0 + 32 * u + (t >> 3), lt = t & 7;
        x[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (rb < total) {
          const int lb = rb / MR, i = rb - lb * MR;
          x[u] = ldg_f4(I.a + ((size_t)i * nb + bb0 + lb) * QK + 4 * lt);
          if (I.lnw) {
            const float m0 = ln[i], v0 = ln[GEMV_MR_MAX + i];
            const size_t e = (size_t)(bb0 + lb) * QK + 4 * lt;
            const float4 w4 = ldg_f4(I.lnw + e), b4 = ldg_f4(I.lnb + e);
            x[u].x = (x[u].x - m0) * v0 * w4.x + b4.x;
            x[u].y = (x[u].y - m0) * v0 * w4.y + b4.y;
            x[u].z = (x[u].z - m0) * v0 * w4.z + b4.z;
            x[u].w = (x[u].w - m0) * v0 * w4.w + b4.w;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        // a wavefront's 8 pairs of pass u start at rb0 + 32 u + 8 (t / 64):
        // passes wholly past the end are skipped (uniform)
        if (U > 4 && rb0 + 32 * u + 8 * (t >> 6) >= total) continue;
        const int rb = rb0 + 32 * u + (t >> 3), lt = t & 7;
        const BlockQuant bq = quantize_block8(x[u]);
        if (rb < total) {
          const int lb = rb / MR, i = rb - lb * MR;
          uint8_t *rec = base + lb * REC;
          *reinterpret_cast<uint32_t *>(rec + 32 * i + mfma_pos(4 * lt)) = pack_q4(bq);
          if (lt == 0) {
            *reinterpret_cast<int *>(rec + SO + 4 * i) = -OFF * bq.sum;
            *reinterpret_cast<float *>(rec + DO + 4 * i) = bq.d;
            *reinterpret_cast<float *>(rec + PO + 4 * i) = __fmul_rn(bq.d, (float)bq.sum);
          }
        }
      }
    }
  } else {
    // already quantized: row group 0 of the activation layout (MFMA order)
    for (int idx = t; idx < total * 8; idx += 256) {
      const int rb = idx >> 3, lt = idx & 7;
      const int lb = rb / MR, i = rb - lb * MR;
      const size_t slot = act_slot(nb, 0, bb0 + lb, i);
      uint8_t *rec = base + lb * REC;
      *reinterpret_cast<uint32_t *>(rec + 32 * i + 4 * lt) = ldg_u32(I.qa + slot * QK + 4 * lt);
      if (lt == 0) {
        *reinterpret_cast<int *>(rec + SO + 4 * i) = -OFF * ldg_i32(I.qsa + slot);
        *reinterpret_cast<float *>(rec + DO + 4 * i) = ldg_f(I.qda + slot);
        *reinterpret_cast<float *>(rec + PO + 4 * i) = ldg_f(I.qpa + slot);
      }
    }
  }
  const int dead = (c1 - c0) * OCT - cnb;
  for (int z = t; z < dead * (REC / 16); z += 256)
    reinterpret_cast<uint4 *>(base + cnb * REC)[z] = make_uint4(0, 0, 0, 0);
}

// Activation records of a grouped decode launch, quantized once per linear
// instead of once per k_gemv workgroup.  8 lanes per (row i, block bl), 4
// elements each (quantize_block8); pairs row-major, so each wavefront reads
// 8 consecutive blocks of a row (1 KB) per load.  Workgroup -> (item, part
// of 32 pairs) through `qwg_item` (item -1 = unused slot).  Each lane writes
// its 4 quants (MFMA order), the block's first lane the row's SEED / DA / PA
// entries, and row 0's first lane also the block's zero parts.  Blocks past
// nb (the padding of the last octet) get zero records.  The values are those
// gemv_fill computes, bit for bit.
template <int DT, int MR>
__global__ __launch_bounds__(256) void k_gemv_records(const GemvItem *__restrict__ items,
                                                      const int2 *__restrict__ qwg_item) {
  constexpr int REC = gemv_rec_bytes(MR), ZO = 32 * MR, SO = ZO + 16, DO = SO + 32, PO = DO + 32;
  constexpr int OFF = DT == 2 ? 8 : DT == 6 ? 16 : 0;
  const int2 wt = qwg_item[blockIdx.x];  // (item, part)
  if (wt.x < 0) return;  // a slot no item uses
  const GemvItem I = items[wt.x];
  const int nb = I.w.nb, nbp = I.w.noct * OCT;
  const int t = threadIdx.x, lt = t & 7;
  const int p = wt.y * 32 + (t >> 3);  // (row, block) pair
  const bool live = p < MR * nbp;      // uniform per 8-lane group
  const int i = p / nbp, bl = p - i * nbp;
  float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
  if (live && bl < nb) x = ldg_f4(I.a + ((size_t)i * nb + bl) * QK + 4 * lt);
  const BlockQuant bq = quantize_block8(x);  // every lane of the wavefront takes part in the DPP moves
  if (!live) return;
  uint8_t *rec = I.rec + (size_t)bl * REC;
  stg_u32(rec + 32 * i + mfma_pos(4 * lt), pack_q4(bq));
  if (lt == 0) {
    stg_u32(rec + SO + 4 * i, (uint32_t)(-OFF * bq.sum));
    stg_f(reinterpret_cast<float *>(rec + DO + 4 * i), bq.d);
    stg_f(reinterpret_cast<float *>(rec + PO + 4 * i), __fmul_rn(bq.d, (float)bq.sum));
    if (i == 0) {
      stg_u4(rec + ZO, make_uint4(0, 0, 0, 0));
#pragma unroll
      for (int r = MR; r < 8; ++r) {
        stg_u32(rec + SO + 4 * r, 0u);
        stg_u32(rec + DO + 4 * r, 0u);
        stg_u32(rec + PO + 4 * r, 0u);
      }
    }
  }
}

// row groups (of 32 weight rows) per k_gemv wavefront: two in grouped
// launches (records shared by more rows), one in single and set launches,
// which are short of workgroups at decode sizes (twice the wavefronts, each
// with half the weight stream, halve their latency)
RW_HD constexpr int gemv_ng(bool grouped) { return grouped ? 2 : 1; }
constexpr int GEMV_NG_MAX = 2;
#ifndef GEMV_WPE
#define GEMV_WPE 4
#endif

// One octet of a wavefront's NG row groups, as loaded: quants (8 bytes,
// Q8_0 16, per lane and block), scales, mins and (Q5) high-bit words.
template <int DT, int NG>
struct GemvOct {
  std::conditional_t<DT == 8, uint4, uint2> q[NG][8];
  uint4 d[NG], m[NG], h0[NG], h1[NG];
};

// (every weight byte is read once per launch: streaming loads)
template <int DT, int NG>
__device__ inline void gemv_load_oct(const WeightView &w, int gw, int o, __amdgpu_buffer_rsrc_t rq,
                                     __amdgpu_buffer_rsrc_t rd, __amdgpu_buffer_rsrc_t rm,
                                     __amdgpu_buffer_rsrc_t rh, uint32_t vq, uint32_t vs, uint32_t vh,
                                     GemvOct<DT, NG> &x) {
  constexpr int QB = DT == 8 ? 32 : 16;
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    const int g = min(gw + j, w.ngroups - 1);
    const uint32_t sq = (uint32_t)(g * w.nb_pad + o * OCT) * (RG * QB);
    const uint32_t ss = (uint32_t)(g * w.noct + o) * (RG * 16);
    x.d[j] = ldb_u4_nt(rd, vs, ss);
    if (has_min(DT)) x.m[j] = ldb_u4_nt(rm, vs, ss);
    if (has_high(DT)) {
      x.h0[j] = ldb_u4_nt(rh, vh, 2 * ss);
      x.h1[j] = ldb_u4_nt(rh, vh + 16, 2 * ss);
    }
#pragma unroll
    for (int b8 = 0; b8 < OCT; ++b8) {
      if constexpr (DT == 8)
        x.q[j][b8] = ldb_u4_nt(rq, vq, sq + b8 * (RG * QB));
      else
        x.q[j][b8] = ldb_u2_nt(rq, vq, sq + b8 * (RG * QB));
    }
  }
}

// Fold one octet into the accumulators: per block and row group one
// v_mfma_i32_32x32x32_i8 (exact sums S of weight rows x activation rows),
// then acc += (d_a*d_b) * S and accm += m_b * (d_a*sum(q_a)) for the
// activation rows 4h..4h+3 this lane holds.  `orec` = the octet's records.
template <int DT, int MR, int NG>
__device__ inline void gemv_fold_oct(const uint8_t *orec, int a_off, int h, int rot, const GemvOct<DT, NG> &x,
                                     float (&acc)[NG][4], float (&accm)[NG][4]) {
  constexpr int REC = gemv_rec_bytes(MR), ZO = 32 * MR, SO = ZO + 16, DO = SO + 32, PO = DO + 32;
  constexpr int OFF = DT == 2 ? 8 : DT == 6 ? 16 : 0;
  constexpr int VR = MR < 4 ? MR : 4;  // rows v of 4h + v that some lane holds
#pragma unroll
  for (int b8 = 0; b8 < OCT; ++b8) {
    const uint8_t *rec = orec + b8 * REC;
    const v4i aop = *reinterpret_cast<const v4i *>(rec + a_off);
    const float4 da = *reinterpret_cast<const float4 *>(rec + DO + 16 * h);
    int4 sd = make_int4(0, 0, 0, 0);
    if (OFF) sd = *reinterpret_cast<const int4 *>(rec + SO + 16 * h);
    const int sdv[4] = {sd.x, sd.y, sd.z, sd.w};
    float4 pa = make_float4(0.f, 0.f, 0.f, 0.f);
    if (has_min(DT)) pa = *reinterpret_cast<const float4 *>(rec + PO + 16 * h);
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      v4i bop;
      if constexpr (DT == 8) {
        const uint4 v = x.q[j][b8];
        bop = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
      } else {
        // low nibbles: elements 8h..8h+7, high nibbles: 16+8h..16+8h+7
        const uint32_t x0 = x.q[j][b8].x, x1 = x.q[j][b8].y;
        uint32_t w0 = x0 & 0x0f0f0f0fu, w1 = x1 & 0x0f0f0f0fu;
        uint32_t w2 = (x0 >> 4) & 0x0f0f0f0fu, w3 = (x1 >> 4) & 0x0f0f0f0fu;
        if (has_high(DT)) {
          const uint32_t hw[8] = {x.h0[j].x, x.h0[j].y, x.h0[j].z, x.h0[j].w,
                                  x.h1[j].x, x.h1[j].y, x.h1[j].z, x.h1[j].w};
          // natural dwords 2h, 2h+1, 4+2h, 5+2h of the block
          const uint32_t xh = __builtin_amdgcn_alignbit(hw[b8], hw[b8], rot);
          w0 |= xh & 0x10101010u;
          w1 |= rotl(xh, 1) & 0x10101010u;
          w2 |= rotl(xh, 4) & 0x10101010u;
          w3 |= rotl(xh, 5) & 0x10101010u;
        }
        bop = v4i{(int)w0, (int)w1, (int)w2, (int)w3};
      }
      const v16i s = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop, v16i{}, 0, 0, 0);
      const uint32_t dw = (b8 >> 1) == 0 ? x.d[j].x : (b8 >> 1) == 1 ? x.d[j].y : (b8 >> 1) == 2 ? x.d[j].z : x.d[j].w;
      const float db = h2f((uint16_t)(dw >> (16 * (b8 & 1))));
      const float dav[4] = {da.x, da.y, da.z, da.w};
      // rows 4h + v: with fewer than 4 rows no lane holds a row v >= MR, so
      // those sums are not folded (they stay 0 and are never stored)
#pragma unroll
      for (int v = 0; v < VR; ++v) acc[j][v] = __builtin_fmaf(dav[v] * db, (float)(s[v] + sdv[v]), acc[j][v]);
      if (has_min(DT)) {
        const uint32_t mw = (b8 >> 1) == 0 ? x.m[j].x : (b8 >> 1) == 1 ? x.m[j].y : (b8 >> 1) == 2 ? x.m[j].z : x.m[j].w;
        const float mb = h2f((uint16_t)(mw >> (16 * (b8 & 1))));
        const float pav[4] = {pa.x, pa.y, pa.z, pa.w};
#pragma unroll
        for (int v = 0; v < VR; ++v) accm[j][v] = __builtin_fmaf(mb, pav[v], accm[j][v]);
      }
    }
  }
}

// Decode shape (m = MR <= 8).  One launch covers any number of linears that
// share (dtype, m); workgroup -> (item, tile) through `wg_item` (GROUPED; item
// -1 = unused slot), or the
// single item `one`: workgroup -> (item, tile of rows).  The host places a
// grouped launch's tiles so that runs of an item's tiles share an XCD, for
// its records to be read through one L2.  The activation rows go to LDS as
// records, copied from
// k_gemv_records' output (GROUPED) or built by gemv_fill, at most `cap_oct`
// octets of blocks at a time.  Each wavefront owns two row
// groups (64 weight rows) and, per block, forms the exact integer sums of
// all its rows against all activation rows with one v_mfma_i32_32x32x32_i8
// per row group: A = the activation block (rows >= MR zero), B = the weight
// block unpacked to int8 in registers (the centered formats' offset enters
// as the seed -c*sum(q_a)).  Lane (r, h) then holds the sums of weight row r
// against activation rows 4h..4h+3 and folds them into f32 accumulators
// exactly as a scalar loop would: acc += (d_a*d_b) * S,
// accm += m_b * (d_a*sum(q_a)).
// 2^lks of the 4 wavefronts split a row's octets (the split depends on the
// weight only); each walks its blocks in increasing order whatever the
// chunking, and the parts meet in LDS in wavefront order: a row's result
// depends on its weight row and activation row alone.  Blocks past nb in the
// last octet meet zero weight planes (the upload writes the padding as
// zeros) and zero activation records: they add exactly +0.
// The epilogue of one lane: y + bias, then GELU (flag 1) and accumulation
// into the output (flag 2), the options the GEMM takes (GEMM_GELU,
// GEMM_ACC).  With PRE, `bv` holds the lane's columns' bias (loaded when
// the tile started); otherwise the bias is loaded here.  Every value the
// epilogue reads is requested before any store, so it costs one memory
// round trip at most.  With PREX the residual values were loaded when the
// tile started as well (`x_in`), so the epilogue reads nothing.
template <int NG>
__device__ inline void gemv_load_residual(const GemvItem &I, int gw, int h, int r, int mr, float (&x)[NG][4]) {
  const int n = I.n;
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    const int col = (gw + j) * RG + r;
#pragma unroll
    for (int v = 0; v < 4; ++v)
      x[j][v] = gw + j < I.w.ngroups && col < n && 4 * h + v < mr ? ldg_f(I.out + (size_t)(4 * h + v) * n + col)
                                                                   : 0.0f;
  }
}
// The records of one block of the outputs a wavefront holds (GEMV_REC_OUT):
// lanes 32 h + r hold column r of block g for rows 4 h + v, so a row's block
// is one half of the wavefront; quantized as quantize_block8 quantizes the
// same 32 values (the largest |x| as integer maxima, NaN skipped, the
// correctly rounded d = amax / 127 and 1 / d, the exact sum of the quants),
// so the records are k_gemv_records' for these rows bit for bit.  Every lane
// of the wavefront calls it (the shuffles); off = the next product's offset
// term (Q4_0 8, Q5_0 16, else 0).
// Over each 32-lane half of the wavefront, in every lane of it: the integer
// maximum (MAX) or the sum, by DPP moves within 16-lane rows (pairs, quads,
// half-row and row mirrors), row 0's (2's) total into row 1 (3) by
// row_bcast:15, and lanes 31 and 63 read back.  Maxima and integer sums are
// exact, so the order does not matter.
template <bool MAX>
__device__ inline int half_reduce32(int v) {
  auto op = [](int a, int b) __attribute__((always_inline)) { return MAX ? max(a, b) : a + b; };
  v = op(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false));   // quad_perm [1,0,3,2]
  v = op(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false));   // quad_perm [2,3,0,1]
  v = op(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false));  // row_half_mirror
  v = op(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xf, 0xf, false));  // row_mirror
  // rows 1 and 3 only (rows 0 and 2 add 0 / take the maximum with 0: values >= 0)
  v = op(v, __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false));  // row_bcast:15
  const int lo = __builtin_amdgcn_readlane(v, 31), hi = __builtin_amdgcn_readlane(v, 63);
  return (threadIdx.x & 32) ? hi : lo;
}

// k_attn's records (several beams' self-attention): the 8 lanes of each
// 8-lane group hold 4 values each of one 32-column block, quantize_block8's
// layout; those with `write` are block bl of row i.  Every lane of the
// wavefront calls it.
__device__ void attn_block_records(uint8_t *rec_base, int i, int bl, int lt, int mr, float4 x, int off, bool write) {
  const int REC = gemv_rec_bytes(mr), ZO = 32 * mr, SO = ZO + 16, DO = SO + 32, PO = DO + 32;
  const BlockQuant bq = quantize_block8(x);
  if (!write) return;
  uint8_t *rec = rec_base + (size_t)bl * REC;
  stg_u32(rec + 32 * i + mfma_pos(4 * lt), pack_q4(bq));
  if (lt == 0) {
    stg_u32(rec + SO + 4 * i, (uint32_t)(-off * bq.sum));
    stg_f(reinterpret_cast<float *>(rec + DO + 4 * i), bq.d);
    stg_f(reinterpret_cast<float *>(rec + PO + 4 * i), __fmul_rn(bq.d, (float)bq.sum));
    if (i == 0) {
      stg_u4(rec + ZO, make_uint4(0, 0, 0, 0));
      for (int z = mr; z < 8; ++z) {
        stg_u32(rec + SO + 4 * z, 0u);
        stg_u32(rec + DO + 4 * z, 0u);
        stg_u32(rec + PO + 4 * z, 0u);
      }
    }
  }
}

// k_attn_combine's records: this lane's output x is element col % 32 of
// block col / 32 of row `row`, and each 32-lane half of the wavefront holds
// one such block; quantized as gemv_records_out quantizes a block.  Every
// lane of the wavefront calls it.
__device__ void combine_records(uint8_t *rec_base, int row, int col, int mr, float x, int off) {
  const int REC = gemv_rec_bytes(mr), ZO = 32 * mr, SO = ZO + 16, DO = SO + 32, PO = DO + 32;
  const int e = col & 31;
  uint8_t *rec = rec_base + (size_t)(col >> 5) * REC;
  const int a = half_reduce32<true>(__float_as_int(fmaxf(fabsf(x), 0.0f)));
  const float d = __fdiv_rn(__int_as_float(a), 127.0f);
  const float inv = d > 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
  const int q = round_clamp_i8(__fmul_rn(x, inv));
  const int sum = half_reduce32<false>(q);
  rec[32 * row + mfma_pos(e)] = (uint8_t)(q & 0xff);
  if (e == 0) {
    stg_u32(rec + SO + 4 * row, (uint32_t)(-off * sum));
    stg_f(reinterpret_cast<float *>(rec + DO + 4 * row), d);
    stg_f(reinterpret_cast<float *>(rec + PO + 4 * row), __fmul_rn(d, (float)sum));
    if (row == 0) {
      stg_u4(rec + ZO, make_uint4(0, 0, 0, 0));
      for (int z = mr; z < 8; ++z) {
        stg_u32(rec + SO + 4 * z, 0u);
        stg_u32(rec + DO + 4 * z, 0u);
        stg_u32(rec + PO + 4 * z, 0u);
      }
    }
  }
}

__device__ inline void gemv_records_out(const GemvItem &I, int g, int h, int r, int mr, const float (&tv)[4],
                                        int off) {
  const int REC = gemv_rec_bytes(mr), ZO = 32 * mr, SO = ZO + 16, DO = SO + 32, PO = DO + 32;
  uint8_t *rec = I.rec + (size_t)g * REC;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    if (v >= mr) break;  // no row 4 h + v of either half (uniform)
    const int a = half_reduce32<true>(__float_as_int(fmaxf(fabsf(tv[v]), 0.0f)));
    const float d = __fdiv_rn(__int_as_float(a), 127.0f);
    const float inv = d > 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    const int q = round_clamp_i8(__fmul_rn(tv[v], inv));
    const int sum = half_reduce32<false>(q);
    const int i = 4 * h + v;
    if (i < mr) {
      rec[32 * i + mfma_pos(r)] = (uint8_t)(q & 0xff);
      if (r == 0) {
        stg_u32(rec + SO + 4 * i, (uint32_t)(-off * sum));
        stg_f(reinterpret_cast<float *>(rec + DO + 4 * i), d);
        stg_f(reinterpret_cast<float *>(rec + PO + 4 * i), __fmul_rn(d, (float)sum));
      }
    }
  }
  if (h == 0 && r == 0) {
    stg_u4(rec + ZO, make_uint4(0, 0, 0, 0));
    for (int z = mr; z < 8; ++z) {
      stg_u32(rec + SO + 4 * z, 0u);
      stg_u32(rec + DO + 4 * z, 0u);
      stg_u32(rec + PO + 4 * z, 0u);
    }
  }
}

// RO: the kernel may be asked for the outputs' records (GEMV_REC_OUT;
// single and set launches of 2-8 rows, the only ones the host asks).
template <bool PRE, int NG, bool PREX, bool RO>
__device__ inline void gemv_epilogue(const GemvItem &I, int gw, int h, int r, int mr, const float (&y)[NG][4],
                                     const float (&bv_in)[NG], const float (&x_in)[NG][4], int off) {
  const int n = I.n;
  float bv[NG], x[NG][4];
#pragma unroll
  for (int j = 0; j < NG; ++j)
    bv[j] = PRE ? bv_in[j] : I.bias ? ldg_f(I.bias + min((gw + j) * RG + r, n - 1)) : 0.0f;
  if (PREX) {
#pragma unroll
    for (int j = 0; j < NG; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) x[j][v] = x_in[j][v];
  } else if (I.flags & 2) {
    gemv_load_residual<NG>(I, gw, h, r, mr, x);
  }
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    const int col = (gw + j) * RG + r;
    if (gw + j < I.w.ngroups && col < n)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (4 * h + v < mr) {
          float t = y[j][v];
          if (I.bias) t = t + bv[j];
          if (I.flags & 1) t = gelu(t);
          if (I.flags & 2) t = x[j][v] + t;
          stg_f(I.out + (size_t)(4 * h + v) * n + col, t);
        }
    if constexpr (RO) {
      // the same values for every lane (the host asks for records only
      // where n is a multiple of 256: every lane's column exists)
      if ((I.flags & GEMV_REC_OUT) && gw + j < I.w.ngroups) {
        float tv[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float t = y[j][v];
          if (I.bias) t = t + bv[j];
          if (I.flags & 1) t = gelu(t);
          if (I.flags & 2) t = x[j][v] + t;
          tv[v] = t;
        }
        gemv_records_out(I, gw + j, h, r, mr, tv, off);
      }
    }
  }
}

// Activation values held in registers by gemv_tile: pair rb = 32 u + t / 8
// of the rows' (block, row) pairs, block-major (the fill's order), lane t % 8
// holding elements 4 (t % 8) .. + 3 of it; NUX passes cover every pair (rows
// of at most 64 blocks, or 160 in the one-row latency form).
//
// Layernorm statistics of the MR rows from those registers: each block's 32
// values summed by its 8 lanes in a fixed tree (DPP), the block sums of a row
// (at most 64, through the start of LDS) then by one wavefront's 64 lanes in
// a fixed tree.  The order depends neither on MR nor on which thread holds a
// block, so a row's mean and inverse deviation are the same bits in every
// launch of every row count.  Mean to ln[i], 1 / sqrt(var + 1e-5) to
// ln[GEMV_MR_MAX + i] (src/tensor.rs:274-287).  All threads call it; it ends
// with a barrier, after which the block sums' LDS is free.
template <int MR, int NUX>
__device__ inline void gemv_ln_stats_regs(const float4 (&xr)[NUX], int nb, uint8_t *lds, int t, float *ln) {
  const int lt = t & 7, l = t & 63, wv = t >> 6;
  const int total = MR * nb;
  const float K = (float)(nb * QK);
  float *sb = reinterpret_cast<float *>(lds);  // [MR][64] block sums
  auto row_sums = [&](auto val, auto fin) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < NUX; ++u) {
      if (32 * u + 8 * wv >= total) continue;  // the wavefront's 8 pairs of pass u are all past the end (uniform)
      const int rb = 32 * u + (t >> 3);
      const int row = rb - (rb / MR) * MR;
      float v = rb < total ? val(u, row) : 0.0f;
      v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));
      v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));
      v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));
      if (rb < total && lt == 0) sb[row * 64 + rb / MR] = v;
    }
    __syncthreads();
    for (int i = wv; i < MR; i += 4) {
      float a = l < nb ? sb[i * 64 + l] : 0.0f;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) a += __shfl_xor(a, o);
      if (l == 0) fin(i, a);
    }
    __syncthreads();
  };
  row_sums([&](int u, int) __attribute__((always_inline)) { return (xr[u].x + xr[u].y) + (xr[u].z + xr[u].w); },
           [&](int i, float a) __attribute__((always_inline)) { ln[i] = __fdiv_rn(a, K); });
  row_sums(
      [&](int u, int row) __attribute__((always_inline)) {
        const float m0 = ln[row];
        const float d0 = xr[u].x - m0, d1 = xr[u].y - m0, d2 = xr[u].z - m0, d3 = xr[u].w - m0;
        return (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
      },
      [&](int i, float a) __attribute__((always_inline)) {
        ln[GEMV_MR_MAX + i] = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(a, K) + 1e-5f));
      });
}

// The records of a one-chunk launch (the whole k in LDS) from the values in
// registers: with I.lnw the rows are layernormed first, (x - mean) * inv * w
// + b as gemv_fill applies it; the quantization is quantize_block8's, so the
// records are gemv_fill's bit for bit.  A block's record goes to the slots
// of the k part that holds its octet (part pp: octets [noct pp >> lks,
// noct (pp+1) >> lks), slots from pp * ch * OCT); the blocks past nb in the
// last octet get zero records.  The slots' parts that no record fills are
// gemv_zero_slots' work.
template <int DT, int MR, int NUX>
__device__ inline void gemv_records_regs(const GemvItem &I, int nb, int noct, int lks, int ch, uint8_t *lds, int t,
                                         const float4 (&xr)[NUX], const float *ln) {
  constexpr int REC = gemv_rec_bytes(MR), SO = 32 * MR + 16, DO = SO + 32, PO = DO + 32;
  constexpr int OFF = DT == 2 ? 8 : DT == 6 ? 16 : 0;
  const int lt = t & 7;
  const int total = MR * nb;
#pragma unroll
  for (int u = 0; u < NUX; ++u) {
    if (32 * u + 8 * (t >> 6) >= total) continue;  // uniform, as in the statistics
    const int rb = 32 * u + (t >> 3);
    const int lb = rb / MR, i = rb - lb * MR;
    float4 x = xr[u];
    if (I.lnw && rb < total) {
      const float m0 = ln[i], v0 = ln[GEMV_MR_MAX + i];
      const size_t e = (size_t)lb * QK + 4 * lt;
      const float4 w4 = ldg_f4(I.lnw + e), b4 = ldg_f4(I.lnb + e);
      x.x = (x.x - m0) * v0 * w4.x + b4.x;
      x.y = (x.y - m0) * v0 * w4.y + b4.y;
      x.z = (x.z - m0) * v0 * w4.z + b4.z;
      x.w = (x.w - m0) * v0 * w4.w + b4.w;
    }
    const BlockQuant bq = quantize_block8(x);  // every lane of the wavefront takes part in its DPP moves
    if (rb < total) {
      const int o = lb >> 3;
      int pp = 0;
#pragma unroll
      for (int q = 1; q < 4; ++q)
        if (q < (1 << lks) && o >= ((noct * q) >> lks)) pp = q;
      uint8_t *rec = lds + ((size_t)pp * ch * OCT + (lb - 8 * ((noct * pp) >> lks))) * REC;
      *reinterpret_cast<uint32_t *>(rec + 32 * i + mfma_pos(4 * lt)) = pack_q4(bq);
      if (lt == 0) {
        *reinterpret_cast<int *>(rec + SO + 4 * i) = -OFF * bq.sum;
        *reinterpret_cast<float *>(rec + DO + 4 * i) = bq.d;
        *reinterpret_cast<float *>(rec + PO + 4 * i) = __fmul_rn(bq.d, (float)bq.sum);
      }
    }
  }
  // the last part's blocks past nb (the tail of its last octet): zero records
  const int pl = (1 << lks) - 1, c0l = (noct * pl) >> lks;
  const int dead = noct * OCT - nb;
  uint4 *dz = reinterpret_cast<uint4 *>(lds + ((size_t)pl * ch * OCT + (nb - 8 * c0l)) * REC);
  for (int z = t; z < dead * (REC / 16); z += 256) dz[z] = make_uint4(0, 0, 0, 0);
}

// One tile of k_gemv: item I's tile wt.y (every wavefront of the workgroup
// calls it; LDS is free on entry and in use on return).  PD > 1: the
// latency form for launches of at most one wavefront per SIMD, whose
// records fit LDS at once: the first PD octets of a wavefront's part are
// requested before the statistics and the fill, and each octet's slot is
// refilled PD octets ahead as soon as it is folded.  The octets are folded
// in the same order whatever PD, so the results do not depend on it.
template <int DT, int MR, bool GROUPED, int PD>
__device__ __attribute__((always_inline)) inline void gemv_tile(const GemvItem I, int2 wt, int cap_oct,
                                                                uint8_t *lds, int lnf = -1) {
  constexpr int REC = gemv_rec_bytes(MR), ZO = 32 * MR;
  constexpr int QB = DT == 8 ? 32 : 16;  // qs bytes per row-block
  constexpr int NG = gemv_ng(GROUPED);
  const WeightView &w = I.w;
  const int nb = w.nb;
  const int lks = I.lks, KS = 1 << lks;
  const int t = threadIdx.x, l = t & 63, h = l >> 5, r = l & 31;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);  // wave-uniform: scalar offsets, uniform loops
  const int set = wv >> lks, part = wv & (KS - 1);
  const int gw = (wt.y * (4 >> lks) + set) * NG;  // first row group
  const int o0 = (w.noct * part) >> lks, o1 = (w.noct * (part + 1)) >> lks;

  // plane buffers (the upload keeps every plane below 4 GiB) and this lane's
  // offsets in them: qs 8 (Q8_0: 16) bytes of row r's block for half h; d,
  // m the row's 8 f16 of an octet; qh its 8 words
  const uint32_t nsc = (uint32_t)w.ngroups * RG * (uint32_t)w.nb_pad;
  const auto rq = buffer_rsrc(w.qs, nsc * QB);
  const auto rd = buffer_rsrc(w.d, nsc * 2);
  const auto rm = buffer_rsrc(w.m, has_min(DT) ? nsc * 2 : 0);
  const auto rh = buffer_rsrc(w.qh, has_high(DT) ? nsc * 4 : 0);
  const uint32_t vq = r * QB + (QB / 2) * h, vs = r * 16, vh = r * 32;
  const int a_off = r < MR ? 32 * r + 16 * h : ZO;
  const int rot = (32 - 2 * h) & 31;  // rotr by this = rotl by 2h

  float acc[NG][4], accm[NG][4];
#pragma unroll
  for (int j = 0; j < NG; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      acc[j][v] = 0.0f;
      accm[j][v] = 0.0f;
    }

  const int span = (w.noct + KS - 1) >> lks;  // the longest part
  // (the latency form holds the whole k: the host launches it only then)
  const int ch = PD > 1 ? span : min(span, max(1, cap_oct >> lks));
  // the first octet's weights are requested before the records and the
  // layernorm statistics (so the memory latencies overlap) where its
  // registers fit beside the fill's: grouped launches copy records and
  // always can; fills can for Q4_0, and for Q4_1 and Q5_0 at one row (the
  // other forms would spill)
  constexpr bool EARLY = PD > 1 || GROUPED || DT == 2 || (MR == 1 && (DT == 3 || DT == 6));
  // Activation values in registers (gemv_ln_stats_regs' layout) for rows of
  // at most 64 blocks: the layernorm statistics come from them, and the
  // latency form at one row (RX) builds its records from them as well, one
  // read of the row instead of two; it requests them with its first weight
  // octets.
  // (the one-row latency form holds rows of up to 160 blocks, k = 5120:
  // the decoder's fc2 input too; statistics from registers need <= 64)
  constexpr bool RX = PD > 1 && !GROUPED && MR == 1;
  constexpr int NUX = GROUPED ? 1 : RX ? 5 : 2 * MR;
  // lnf: whether the rows are layernormed, when the caller knows it without
  // reading the item (-1: from I.lnw)
  const bool has_ln = lnf >= 0 ? lnf != 0 : I.lnw != nullptr;
  const bool stats_regs = !GROUPED && I.a != nullptr && nb <= 64 && has_ln;  // uniform
  const bool regs = RX && I.a != nullptr && nb <= 32 * NUX;
  const bool xin = stats_regs || regs;
  // the outputs' records for a next product (GEMV_REC_OUT), and its offset term
  constexpr bool RO = !GROUPED && MR > 1;
  constexpr int OFFR = DT == 2 ? 8 : DT == 6 ? 16 : 0;
  // records written by the previous product's epilogue (GEMV_REC_OUT) are
  // copied whole, as a grouped launch copies k_gemv_records' output
  // (2-8 rows only, as the host passes them)
  const bool rin = !GROUPED && MR > 1 && I.a == nullptr && I.rec != nullptr;  // uniform
  // the latency form requests them with its first octets when that needs
  // nothing from the argument block (lnf known)
  const bool x_early = PD > 1 && xin && (regs || lnf >= 0);
  float4 xr[NUX];
  auto load_x = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < NUX; ++u) {
      const int rb = 32 * u + (t >> 3);
      xr[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (rb < MR * nb) {
        const int lb = rb / MR, i = rb - lb * MR;
        xr[u] = ldg_f4(I.a + ((size_t)i * nb + lb) * QK + 4 * (t & 7));
      }
    }
  };
  GemvOct<DT, NG> ring[PD];
  GemvOct<DT, NG> &cur = ring[0];
  if (EARLY) {
#pragma unroll
    for (int u = 0; u < PD; ++u)
      if (o0 + u < min(o1, o0 + ch)) gemv_load_oct<DT, NG>(w, gw, o0 + u, rq, rd, rm, rh, vq, vs, vh, ring[u]);
  }
  if (x_early) load_x();
  // grouped launches: this lane's columns' bias, in flight with the first
  // octet (the others, and Q5_1, load it in the epilogue: registers)
  // The latency form (PD > 1) also requests the residual values of the
  // epilogue here (flag 2; nothing in the launch writes them before the
  // epilogue), so its end costs no memory round trip.
  constexpr bool PRE = (GROUPED && DT != 7) || PD > 1, PREX = PD > 1;
  float bv[NG], xres[NG][4];
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    bv[j] = PRE && I.bias && part == 0 ? ldg_f(I.bias + min((gw + j) * RG + r, I.n - 1)) : 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) xres[j][v] = 0.0f;
  }
  if (PREX && part == 0 && (I.flags & 2)) gemv_load_residual<NG>(I, gw, h, r, MR, xres);

  // layernorm statistics of the m activation rows (single / set launches
  // with I.lnw): every workgroup computes them, in the same tree order, and
  // keeps them in LDS for the fills; rows of at most 64 blocks from the
  // values in registers (fixed per-block and per-row trees), longer rows by
  // the loop below
  __shared__ float ln_s[2 * GEMV_MR_MAX];
  if constexpr (!GROUPED) {
    if (stats_regs) {
      if (!x_early) load_x();
      gemv_ln_stats_regs<MR, NUX>(xr, nb, lds, t, ln_s);
    } else if (has_ln) {
      const int K = nb * QK;
      float *sred = reinterpret_cast<float *>(lds);  // [4 wavefronts][MR], before any record
      auto row_sums = [&](float (&v)[MR]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < MR; ++i) {
          float a = v[i];
#pragma unroll
          for (int o = 1; o < 64; o <<= 1) a += __shfl_xor(a, o);
          if (l == 0) sred[wv * MR + i] = a;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < MR; ++i) v[i] = (sred[i] + sred[MR + i]) + (sred[2 * MR + i] + sred[3 * MR + i]);
        __syncthreads();
      };
      // a thread's values of a row, c = t, t + 256, ..., summed in that
      // order; loaded 8 at a time so that their latencies overlap
      auto thread_sum = [&](const float *row, float mu, bool sq) __attribute__((always_inline)) {
        float a = 0.0f;
        for (int c0 = t; c0 < K; c0 += 8 * 256) {
          float v[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) v[u] = c0 + 256 * u < K ? row[c0 + 256 * u] : 0.0f;
#pragma unroll
          for (int u = 0; u < 8; ++u)
            if (c0 + 256 * u < K) {
              const float d = v[u] - mu;
              a += sq ? d * d : v[u];
            }
        }
        return a;
      };
      float acc_s[MR], mean[MR];
#pragma unroll
      for (int i = 0; i < MR; ++i) acc_s[i] = thread_sum(I.a + (size_t)i * K, 0.0f, false);
      row_sums(acc_s);
#pragma unroll
      for (int i = 0; i < MR; ++i) {
        mean[i] = __fdiv_rn(acc_s[i], (float)K);
        acc_s[i] = thread_sum(I.a + (size_t)i * K, mean[i], true);
      }
      row_sums(acc_s);
      if (t == 0) {
#pragma unroll
        for (int i = 0; i < MR; ++i) {
          ln_s[i] = mean[i];
          ln_s[GEMV_MR_MAX + i] = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(acc_s[i], (float)K) + 1e-5f));
        }
      }
      __syncthreads();
    }
  }

  // zero the parts of every record slot the fills never write (records
  // copied whole need none); after the statistics, whose partial sums use
  // the start of LDS
  if (!GROUPED) gemv_zero_slots<MR>(lds, cap_oct * OCT, t);

  // chunks: step cc covers octets [s_p + cc, s_p + cc + ch) of every part
  // p (s_p its first octet), in LDS slots [p*ch, (p+1)*ch), so that every
  // part advances through every chunk
  for (int cc = 0; cc < span; cc += ch) {
    // this part's octets in the chunk
    const int p0 = o0 + cc, p1 = min(o1, p0 + ch);
    if (EARLY && cc && p0 < p1) gemv_load_oct<DT, NG>(w, gw, p0, rq, rd, rm, rh, vq, vs, vh, cur);
    if (cc) __syncthreads();  // every wavefront is done with the previous chunk
    for (int pp = 0; pp < KS; ++pp) {
      const int c0 = ((w.noct * pp) >> lks) + cc, c1 = min((w.noct * (pp + 1)) >> lks, c0 + ch);
      if (c0 >= c1) continue;
      uint8_t *base = lds + pp * ch * OCT * REC;
      if (GROUPED || rin) {
        // RB loads per thread in flight at a time (as many as the
        // registers beside the first octet's allow)
        constexpr int RB = DT == 2 || DT == 6 ? 4 : DT == 7 ? 1 : 2;
        const uint4 *src = reinterpret_cast<const uint4 *>(I.rec + (size_t)c0 * OCT * REC);
        const int total = (c1 - c0) * OCT * (REC / 16);
        for (int z0 = t; z0 < total; z0 += RB * 256) {
          uint4 rv[RB];
#pragma unroll
          for (int u = 0; u < RB; ++u)
            if (z0 + 256 * u < total) rv[u] = ldg_u4(src + z0 + 256 * u);
#pragma unroll
          for (int u = 0; u < RB; ++u)
            if (z0 + 256 * u < total) reinterpret_cast<uint4 *>(base)[z0 + 256 * u] = rv[u];
        }
      } else if (!regs) {
        gemv_fill<DT, MR, (PD > 1 && MR == 1 ? 8 : 4)>(I, nb, c0, c1, base, t, ln_s);
      }
    }
    if constexpr (RX) {
      if (regs) gemv_records_regs<DT, MR, NUX>(I, nb, w.noct, lks, ch, lds, t, xr, ln_s);
    }
    __syncthreads();

    // --- weights: each octet loaded whole for all row groups (the planes
    // are padded to whole octets), then folded in
    if (p0 < p1) {
      if constexpr (PD > 1) {  // one chunk: octets p0 .. p0 + PD - 1 are in flight
        for (int o = p0; o < p1; o += PD) {
#pragma unroll
          for (int u = 0; u < PD; ++u)
            if (o + u < p1) {
              gemv_fold_oct<DT, MR, NG>(lds + (part * ch + o + u - p0) * OCT * REC, a_off, h, rot, ring[u], acc, accm);
              if (o + u + PD < p1) gemv_load_oct<DT, NG>(w, gw, o + u + PD, rq, rd, rm, rh, vq, vs, vh, ring[u]);
            }
        }
      } else {
        if (!EARLY) gemv_load_oct<DT, NG>(w, gw, p0, rq, rd, rm, rh, vq, vs, vh, cur);
        gemv_fold_oct<DT, MR, NG>(lds + part * ch * OCT * REC, a_off, h, rot, cur, acc, accm);
        for (int o = p0 + 1; o < p1; ++o) {
          gemv_load_oct<DT, NG>(w, gw, o, rq, rd, rm, rh, vq, vs, vh, cur);
          gemv_fold_oct<DT, MR, NG>(lds + (part * ch + o - p0) * OCT * REC, a_off, h, rot, cur, acc, accm);
        }
      }
    }
  }

  float y[NG][4];
#pragma unroll
  for (int j = 0; j < NG; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) y[j][v] = has_min(DT) ? acc[j][v] + accm[j][v] : acc[j][v];

  if (KS == 1) {
    gemv_epilogue<PRE, NG, PREX, RO>(I, gw, h, r, MR, y, bv, xres, OFFR);
    return;
  }
  __syncthreads();  // the activation LDS is reused for the partial sums
  float *red = reinterpret_cast<float *>(lds);  // [4 wavefronts][NG groups x 4][64]
#pragma unroll
  for (int j = 0; j < NG; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[(wv * 4 * NG + 4 * j + v) * 64 + l] = y[j][v];
  __syncthreads();
  if (part == 0) {
#pragma unroll
    for (int j = 0; j < NG; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float tt = red[(wv * 4 * NG + 4 * j + v) * 64 + l];
        for (int p = 1; p < KS; ++p) tt = tt + red[((wv + p) * 4 * NG + 4 * j + v) * 64 + l];
        y[j][v] = tt;
      }
    gemv_epilogue<PRE, NG, PREX, RO>(I, gw, h, r, MR, y, bv, xres, OFFR);
  }
}

// One launch: workgroup -> (item, tile) through `wg_item` (grouped; item -1
// = an unused slot) or, for a single or set launch, the set's item by
// uniform compares (no runtime index into the argument).
// The leading arguments repeat what the first item's tiles need before
// their first memory requests (its activation rows, weight planes and
// geometry; hdr = set count | lks << 4 | layernorm << 6 | cap_oct << 8)
// as plain scalars:
// the first 14
// dwords of a launch's arguments arrive in SGPRs when its waves start
// (kernarg preloading), so a single linear's tiles request their rows and
// weights without waiting for the argument block (GemvSet) to be read;
// grouped launches pass zeros.
template <int DT, int MR, bool GROUPED, int PD = 1>
__global__ __launch_bounds__(256, PD > 1 ? 1 : GEMV_WPE) void k_gemv(
    const float *a0, const uint8_t *qs0, const uint16_t *d0, const uint32_t *qh0, const uint16_t *m0, int nb0,
    int noct0, int ngroups0, int hdr, const GemvItem *__restrict__ items, const int2 *__restrict__ wg_item,
    GemvSet one, int cap_oct) {
  extern __shared__ __align__(16) uint8_t lds[];
  // the descriptor is wave-uniform: scalar loads from the table or kernarg
  if constexpr (GROUPED) {
    const int2 wt = wg_item[blockIdx.x];  // (item, tile)
    if (wt.x < 0) return;                 // a slot no item uses (the whole workgroup)
    gemv_tile<DT, MR, true, PD>(items[wt.x], wt, cap_oct, lds);
  } else {
    if ((hdr & 15) == 1) {
      // one linear: its early fields from the leading scalars, so that no
      // value merged from another item waits for the argument block's loads
      GemvItem I = one.it[0];
      I.a = a0;
      I.w.qs = qs0;
      I.w.d = d0;
      I.w.qh = qh0;
      I.w.m = m0;
      I.w.nb = nb0;
      I.w.noct = noct0;
      I.w.nb_pad = noct0 * OCT;
      I.w.ngroups = ngroups0;
      I.lks = (hdr >> 4) & 3;
      gemv_tile<DT, MR, false, PD>(I, make_int2(0, (int)blockIdx.x), (hdr >> 8) & 255, lds, (hdr >> 6) & 1);
    } else {
      // a set: the workgroup's item by uniform compares (its end[] entries
      // and fields from the argument block; measured faster than reading
      // the item at a computed offset)
      int ii = 0;
#pragma unroll
      for (int t = 0; t + 1 < GEMV_SET; ++t)
        if (t + 1 < one.count && (int)blockIdx.x >= one.end[t]) ii = t + 1;
      int first = 0;
#pragma unroll
      for (int t = 0; t + 1 < GEMV_SET; ++t)
        if (ii == t + 1) first = one.end[t];
      GemvItem I = one.it[0];
#pragma unroll
      for (int t = 1; t < GEMV_SET; ++t)
        if (ii == t) I = one.it[t];
      gemv_tile<DT, MR, false, PD>(I, make_int2(ii, (int)blockIdx.x - first), cap_oct, lds);
    }
  }
}

// LDS bytes k_gemv needs for m rows and cap_oct octets of records
RW_HD inline size_t gemv_lds_bytes(int m, int cap_oct) {
  const size_t act = (size_t)cap_oct * OCT * gemv_rec_bytes(m);
  const size_t red = (size_t)4 * 4 * GEMV_NG_MAX * 64 * 4;
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

// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector
// memory operations of this wavefront are outstanding, nothing else
RW_HD constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }


// One lane's operands of one block of k_gemm: A (its 16-byte chunk of each
// of the two MFMAs, for TM activation row groups) and B raw (its 16 quant
// bytes and the block's (d, m), for TN weight row groups).
template <int TM, int TN>
struct GemmStage {
  uint4 a[TM][2];
  uint4 q[TN];
  uint32_t dm[TN];
};
template <int TN>
struct GemmB {
  v8h b[TN][2];
};

// B operands of one block for lane half h: the 16 quant bytes (MFMA order)
// -> exact centered quants in f16 -> f16(d_b * q_b + m_b), one rounding
template <int DT>
__device__ inline void weight_f16(uint4 qb, uint32_t dmw, v8h &b0, v8h &b1) {
  uint32_t q[4] = {qb.x, qb.y, qb.z, qb.w};
  if (DT == 8) {
#pragma unroll
    for (int t = 0; t < 4; ++t) q[t] ^= 0x80808080u;
  }
  v8h q0, q1;
  quants_to_f16<DT>(q, q0, q1);
  const h2v dmh = __builtin_bit_cast(h2v, dmw);
  const v8h dv = dmh.x, mv = dmh.y;
  b0 = __builtin_elementwise_fma(q0, dv, mv);
  b1 = __builtin_elementwise_fma(q1, dv, mv);
}

constexpr int GEMM_TN = 2, GEMM_P = 2;
// blocks in flight for 64-row tiles (skinny launches: a few wavefronts
// per column tile, each a chain of block loads, so latency-bound)
#ifndef GEMM_P_SKINNY
#define GEMM_P_SKINNY 4
#endif

// The weights of one k_gemm launch (all of one dtype and k, against one
// quantized activation): column tiles [tile0, tile0 + cdiv(ngroups, TN)) of
// the launch belong to item i.
constexpr int GEMM_MAX_SET = 4;
// epilogue options of a GEMM item: GELU (tanh form, src/tensor.rs:289-305)
// on y = x W^T + b, and accumulation into the output (out += y, the
// residual add of src/encoder.rs:146-148, 171-173)
constexpr int GEMM_GELU = 1, GEMM_ACC = 2;
// GEMM_QUANT: instead of the f32 output, quantize_acts_i8 of each output row
// block (32 columns of a 32 x 32 tile): the int8 quants into qo and each
// block's largest |y| into ao, both by (row group, block) as the tiles
// produce them -- qo [mgroups][n / 32][32 rows][32], ao [mgroups][n / 32][32
// rows] -- from which k_quantize_finish builds the next product's f16
// operand (n % 32 == 0)
constexpr int GEMM_QUANT = 4;
struct GemmItem {
  GemmPlanes gp;
  const float *bias;
  float *out;
  int8_t *qo;
  float *ao;
  int n, ngroups, tile0, flags;
};


struct GemmSet {
  GemmItem it[GEMM_MAX_SET];
  int count, nb, nb_pad;
};

// Encoder-shape GEMM (m > 8): out = rs * (A' W'^T) * cs + cm * ps (+ bias),
// with A' the f16 values of the quantized activations (k_quantize_f16), ps
// their exact row sums, and W' = f16((d_b*q_b + m_b - cm) / cs) formed in
// registers from the byte plane with one packed f16 fma per two weights (a
// single rounding; cs and cm are the weight row's power of two and offset,
// so W' never overflows and rounds relative to the row's spread).  Products
// of f16 operands are exact and accumulate in f32 inside
// v_mfma_f32_32x32x16_f16, so |y - exact| <= 2^-10 sum|a||w - cm| plus the
// f32 accumulation error.
// A launch covers up to GEMM_MAX_SET weights that share the activation (the
// column tiles of the launch run through the weights in turn).  A
// workgroup owns one tile of TM activation row groups x TN weight row
// groups (32 TM x 32 TN; TM = 4, 3 or 2, TN = 2, or 1 for skinny inputs,
// whose launches are short of wavefronts) and has KW wavefronts, each
// taking every KW-th block
// (block kw, kw + KW, ...).  A wavefront loads its operands straight into
// registers, P blocks ahead, and needs no other wavefront until the end: no
// LDS and no barrier in the k loop.  Each step issues the loads of block
// s + P, then runs the 16 MFMAs of block s while the VALU dequantizes the
// weights of block s + 1 (one MFMA, then three VALU instructions).  At the
// end the KW partial tiles meet in LDS and are summed in kw order, the
// 32 x 32 output tiles dealt to the wavefronts in turn.  KW comes from the
// weights' shapes alone and TM changes which rows share a workgroup, not
// how a row is summed, so a row's result never depends on m.
// One workgroup's tile of k_gemm: item `it`'s column tile bx (of its own
// weight) against activation row tile by.
template <int DT, int KW, int TM, bool OFFS, int TN>
__device__ __attribute__((always_inline)) inline void gemm_tile(const GemmItem &it, const ActView &a, int nb,
                                                                int nb_pad, int m, int bx, int by, uint8_t *lds) {
  constexpr int P = TM <= 2 ? GEMM_P_SKINNY : GEMM_P, S = P + 1;
  constexpr int RED = KW > 1 ? KW * TM * TN * 16 * 64 * 4 : 16;
  constexpr int QROW = 36;  // floats per row of a GEMM_QUANT staging tile (rows 4 apart on other banks)
  const int l = threadIdx.x & 63;
  const int kw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = l >> 5, r = l & 31;
  const GemmPlanes gp = it.gp;
  const float *__restrict__ bias = it.bias;
  float *__restrict__ out = it.out;
  const int n = it.n, ngroups = it.ngroups, flags = it.flags;
  
  const int nsw = nb > kw ? (nb - kw + KW - 1) / KW : 0;  // this wavefront's block count

  // operands through buffer loads: one resource per plane, a constant lane
  // offset per row group, and the block's offset in a scalar register (no
  // per-lane address arithmetic in the loop); row groups past the end repeat
  // the last one
  const auto ra = buffer_rsrc(a.a16, (uint32_t)a.mgroups * (uint32_t)nb * 2048u);
  const auto rq = buffer_rsrc(gp.q8, (uint32_t)ngroups * (uint32_t)nb_pad * 1024u);
  const auto rd = buffer_rsrc(gp.dm, (uint32_t)ngroups * (uint32_t)nb_pad * 128u);
  uint32_t aoff[TM], qoff[TN], doff[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) aoff[i] = (uint32_t)min(by * TM + i, a.mgroups - 1) * (uint32_t)nb * 2048u + l * 16;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const uint32_t g = (uint32_t)min(bx * TN + j, ngroups - 1);
    qoff[j] = g * (uint32_t)nb_pad * 1024u + r * 32 + 16 * h;
    doff[j] = g * (uint32_t)nb_pad * 128u + r * 4;
  }
  auto load = [&](GemmStage<TM, TN> &st, int s) __attribute__((always_inline)) {
    const uint32_t bl = (uint32_t)(kw + s * KW);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      st.a[i][0] = ldb_u4(ra, aoff[i], bl * 2048u);
      st.a[i][1] = ldb_u4(ra, aoff[i] + 1024, bl * 2048u);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      st.q[j] = ldb_u4(rq, qoff[j], bl * 1024u);
      st.dm[j] = ldb_u32(rd, doff[j], bl * 128u);
    }
  };
  auto deq = [&](const GemmStage<TM, TN> &st) __attribute__((always_inline)) {
    GemmB<TN> o;
#pragma unroll
    for (int j = 0; j < TN; ++j) weight_f16<DT>(st.q[j], st.dm[j], o.b[j][0], o.b[j][1]);
    return o;
  };
  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (v16f){};
  auto mma = [&](const GemmStage<TM, TN> &st, const GemmB<TN> &b) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, st.a[i][0]), b.b[j][0],
                                                           acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, st.a[i][1]), b.b[j][1],
                                                           acc[i][j], 0, 0, 0);
      }
  };

  // loads never pass this wavefront's last block: later stages re-read it
  GemmStage<TM, TN> st[S];
#pragma unroll
  for (int u = 0; u < P; ++u) load(st[u], min(u, max(nsw - 1, 0)));
  GemmB<TN> bc = deq(st[0]);
  int s = 0;
  for (; s + S <= nsw; s += S) {
#pragma unroll
    for (int u = 0; u < S; ++u) {
      __builtin_amdgcn_sched_barrier(0);
      load(st[(u + P) % S], min(s + u + P, nsw - 1));
      __builtin_amdgcn_sched_barrier(0);
      const GemmB<TN> bn = deq(st[(u + 1) % S]);
      mma(st[u], bc);
#pragma unroll
      for (int k = 0; k < 2 * TM * TN; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // three VALU
      }
      __builtin_amdgcn_sched_barrier(0);
      bc = bn;
    }
  }
  // The workgroup's TM x TN output tiles (32 x 32 each, tile u = TN i + j)
  // are dealt to the KW wavefronts in runs of UPW: a wavefront finishes RPW
  // row groups x CPW column groups (whole rows of tiles, or UPW tiles of one
  // row).  Their epilogue inputs are requested before the last blocks' MFMAs
  // and land while those run and the partials meet in LDS (rows and columns
  // past the end read the last one).
  constexpr int NU = TM * TN, UPW = (NU + KW - 1) / KW;
  static_assert(UPW >= TN ? UPW % TN == 0 : TN % UPW == 0, "a run covers whole rows of tiles or part of one");
  constexpr int RPW = UPW >= TN ? UPW / TN : 1, CPW = UPW >= TN ? TN : UPW;
  const int u0 = KW > 1 ? kw * UPW : 0;  // first tile of this wavefront
  const int i0 = u0 / TN, j0 = UPW >= TN ? 0 : u0 % TN;
  // OFFS: some weight of the launch has rows with an offset (GemmPlanes::cm;
  // a weight without one has cm == NULL and reads 0)
  const bool offs = OFFS && gp.cm != nullptr;  // uniform
  const float *bp = bias ? bias : gp.cs;
  const float *cmp = offs ? gp.cm : gp.cs;
  float4 sc[RPW][4], pv[RPW][4];
  float bv[CPW], cv[CPW], mv[CPW];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const int tg = min(by * TM + min(i0 + rr, TM - 1), a.mgroups - 1);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      sc[rr][q] = ldg_f4(a.rs + tg * RG + 8 * q + 4 * h);
      if (OFFS) pv[rr][q] = ldg_f4(a.ps + tg * RG + 8 * q + 4 * h);
    }
  }
#pragma unroll
  for (int cc = 0; cc < CPW; ++cc) {
    const int cg = min(bx * TN + j0 + cc, ngroups - 1), wr = cg * RG + r;  // padding rows: cs 1, cm 0
    bv[cc] = ldg_f(bp + (bias ? min((bx * TN + j0 + cc) * RG + r, n - 1) : wr));
    cv[cc] = ldg_f(gp.cs + wr);
    if (OFFS) mv[cc] = offs ? ldg_f(cmp + wr) : 0.0f;
  }
  // GEMM_ACC: the output values this wavefront adds to, requested here with
  // the other epilogue inputs where they fit (at most 2 tiles: 32 values per
  // lane), so no load waits behind the epilogue's stores (stores count in
  // the same counter); only this wavefront touches its tiles' outputs
  constexpr bool XPRE = RPW * CPW <= 2;
  float xpre[XPRE ? RPW : 1][XPRE ? CPW : 1][16];
  auto load_res = [&](int rr, int cc, float (&x)[16]) __attribute__((always_inline)) {
    const int tg = by * TM + i0 + rr, cg = bx * TN + j0 + cc, col = cg * RG + r;
    const bool ok = tg < a.mgroups && cg < ngroups && col < n;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int row = tg * RG + 4 * h + 8 * (v >> 2) + (v & 3);
      x[v] = ok && row < m ? ldg_f(out + (size_t)row * n + col) : 0.0f;
    }
  };
  if (XPRE && (flags & GEMM_ACC)) {
#pragma unroll
    for (int rr = 0; rr < (XPRE ? RPW : 1); ++rr)
#pragma unroll
      for (int cc = 0; cc < (XPRE ? CPW : 1); ++cc) load_res(rr, cc, xpre[rr][cc]);
  }
  // the last nsw - s (< S) blocks are already in st[0 ..]
#pragma unroll
  for (int u = 0; u < S - 1; ++u)
    if (s + u < nsw) {
      const GemmB<TN> bn = deq(st[(u + 1) % S]);
      mma(st[u], bc);
      bc = bn;
    }

  float4 *red = reinterpret_cast<float4 *>(lds);
  if (KW > 1) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          red[(((kw * TM + i) * TN + j) * 4 + q) * 64 + l] =
              make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
    __syncthreads();
  }
  // every epilogue load has landed before the first store: stores count in
  // the same counter, and a wait placed behind them would wait for them
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  if (u0 >= NU) return;  // a wavefront with no tile of its own (after the barrier)
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr)
#pragma unroll
  for (int cc = 0; cc < CPW; ++cc) {
    const int i = i0 + rr, j = j0 + cc;  // compile-time with one wavefront
    const int tg = by * TM + i, cg = bx * TN + j;
    if (tg >= a.mgroups || cg >= ngroups) continue;
    const bool rows_full = (tg + 1) * RG <= m;
    const int col = cg * RG + r;
    float y[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float4 v;
      if constexpr (KW > 1) {
        v = red[((i * TN + j) * 4 + q) * 64 + l];
#pragma unroll
        for (int kk = 1; kk < KW; ++kk) {
          const float4 p = red[(((kk * TM + i) * TN + j) * 4 + q) * 64 + l];
          v.x += p.x;
          v.y += p.y;
          v.z += p.z;
          v.w += p.w;
        }
      } else {
        v = make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
      }
      // row scale, then column scale: both powers of two, so exact (the
      // row scale first keeps the intermediate in range); then the weight
      // row's offset times the activation row's sum, one rounding
      const float4 c = sc[rr][q];
      y[4 * q] = (v.x * c.x) * cv[cc];
      y[4 * q + 1] = (v.y * c.y) * cv[cc];
      y[4 * q + 2] = (v.z * c.z) * cv[cc];
      y[4 * q + 3] = (v.w * c.w) * cv[cc];
      if (OFFS && offs) {
        const float4 pp = pv[rr][q];
        y[4 * q] = __builtin_fmaf(mv[cc], pp.x, y[4 * q]);
        y[4 * q + 1] = __builtin_fmaf(mv[cc], pp.y, y[4 * q + 1]);
        y[4 * q + 2] = __builtin_fmaf(mv[cc], pp.z, y[4 * q + 2]);
        y[4 * q + 3] = __builtin_fmaf(mv[cc], pp.w, y[4 * q + 3]);
      }
      if (bias) {
#pragma unroll
        for (int e = 0; e < 4; ++e) y[4 * q + e] += bv[cc];
      }
    }
    if (flags & GEMM_GELU) {
#pragma unroll
      for (int v = 0; v < 16; ++v) y[v] = gelu(y[v]);
    }
    if (flags & GEMM_QUANT) {
      // The tile's 32 columns are one block of each of its 32 rows in the
      // next product's input.  Through this wavefront's LDS tile, 8 lanes
      // take a (row, block) with 4 elements each and quantize it as
      // quantize_block8 (and k_quantize_f16) does.  A wavefront's LDS
      // accesses complete in order, so its lanes read what the others wrote.
      float *stg = reinterpret_cast<float *>(lds + RED) + kw * (32 * QROW);
#pragma unroll
      for (int v = 0; v < 16; ++v) stg[(8 * (v >> 2) + 4 * h + (v & 3)) * QROW + r] = y[v];
      const int lb = l >> 3, lt = l & 7;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int rw = lb + 8 * u, row = tg * RG + rw;
        const float4 xv = *reinterpret_cast<const float4 *>(stg + rw * QROW + 4 * lt);
        const float amax = max8_nn(amax4(xv));
        const float d = __fdiv_rn(amax, 127.0f);
        const float inv = d > 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
        const uint32_t q = (uint32_t)(round_clamp_i8(__fmul_rn(xv.x, inv)) & 0xff) |
                           ((uint32_t)(round_clamp_i8(__fmul_rn(xv.y, inv)) & 0xff) << 8) |
                           ((uint32_t)(round_clamp_i8(__fmul_rn(xv.z, inv)) & 0xff) << 16) |
                           ((uint32_t)(round_clamp_i8(__fmul_rn(xv.w, inv)) & 0xff) << 24);
        if (row < m) {
          const size_t slot = ((size_t)tg * (size_t)(n / RG) + cg) * RG + rw;
          stg_u32(it.qo + slot * QK + 4 * lt, q);
          if (lt == 0) stg_f(it.ao + slot, amax);
        }
      }
      continue;
    }
    if (flags & GEMM_ACC) {
      // x + y: the tile's 16 values loaded (early, or all before any store)
      float x[16];
      if constexpr (XPRE) {
#pragma unroll
        for (int v = 0; v < 16; ++v) x[v] = xpre[XPRE ? rr : 0][XPRE ? cc : 0][v];
      } else {
        load_res(rr, cc, x);
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) y[v] = x[v] + y[v];
    }
    // lane (h, r) holds rows 8q + 4h + e (e < 4) of column col
    float *o = out + (size_t)(tg * RG + 4 * h) * n + col;
    if (rows_full && (cg + 1) * RG <= n) {
#pragma unroll
      for (int v = 0; v < 16; ++v) stg_f(o + (size_t)(8 * (v >> 2) + (v & 3)) * n, y[v]);
    } else if (col < n) {
#pragma unroll
      for (int v = 0; v < 16; ++v)
        if (tg * RG + 4 * h + 8 * (v >> 2) + (v & 3) < m) stg_f(o + (size_t)(8 * (v >> 2) + (v & 3)) * n, y[v]);
    }
  }
}

// The leading arguments repeat the activation plane, the first weight's
// planes and the launch's geometry (hdr = the set's count; nx, ny = the
// grid) as plain
// scalars: the first 14 dwords arrive in SGPRs when the waves start
// (kernarg preloading), so a one-weight launch requests its first operand
// blocks without first reading the argument block.
template <int DT, int KW, int TM, bool OFFS, int TN = GEMM_TN>
__global__ __launch_bounds__(64 * KW, 1) void k_gemm(const uint16_t *a16, const uint8_t *q80, const uint32_t *dm0,
                                                      int nb, int nb_pad, int mgroups, int ngroups0, int m, int hdr,
                                                      int nx, int ny, GemmSet set, ActView a) {
  constexpr int RED = KW > 1 ? KW * TM * TN * 16 * 64 * 4 : 16;
  constexpr int QROW = 36;
  __shared__ __align__(16) uint8_t lds[RED + KW * 32 * QROW * 4];
  int bx, by;
  {
    // XCD-aware order: consecutive workgroup ids go to different XCDs (id % 8);
    // each XCD gets one contiguous band of the row-major tile order, so its
    // L2 holds one band of activation rows.
    const int total = nx * ny;  // the grid (gridDim would be read from the argument block)
    const int id = blockIdx.y * nx + blockIdx.x;
    const int per = total / 8, rem = total % 8, xcd = id % 8, slot = id / 8;
    const int lin = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
    bx = lin % nx;
    by = lin / nx;
  }
  ActView av = a;
  av.a16 = a16;
  av.mgroups = mgroups;
  av.nb = nb;
  if (hdr == 1) {
    GemmItem it = set.it[0];
    it.gp.q8 = q80;
    it.gp.dm = dm0;
    it.ngroups = ngroups0;
    gemm_tile<DT, KW, TM, OFFS, TN>(it, av, nb, nb_pad, m, bx, by, lds);
  } else {
    // this tile's weight, selected by uniform compares (no runtime index
    // into the argument array)
    int wi = 0;
#pragma unroll
    for (int t = 1; t < GEMM_MAX_SET; ++t)
      if (t < hdr && bx >= set.it[t].tile0) wi = t;
    GemmItem it = set.it[0];
#pragma unroll
    for (int t = 1; t < GEMM_MAX_SET; ++t)
      if (wi == t) it = set.it[t];
    gemm_tile<DT, KW, TM, OFFS, TN>(it, av, nb, nb_pad, m, bx - it.tile0, by, lds);
  }
}

}  // namespace rw
