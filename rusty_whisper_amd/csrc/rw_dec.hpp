// rw_dec.hpp -- the small element-wise kernels of the decoder step (device
// code): the token + position embedding, a float32 layernorm (with the
// residual add of src/decoder.rs:168-170, 191-193 and mlp_block folded in
// front of it) and GELU.  The products and attention are the kernels of
// rw_kernels.hpp and rw_attn.hpp.
#pragma once
#include <stdint.h>

#include "rw_layout.hpp"

namespace rw {

#if defined(__HIPCC__)

// x[i] = token_embedding.row_f32(tok[i]) + positional[n_past + i]
// (src/decoder.rs:122-135): the quantized row dequantized as d * q + m (two
// roundings), then the position added.  One thread per (token, block).
template <int DT>
__global__ __launch_bounds__(256) void k_embed(WeightView w, const int *__restrict__ tok, int n_tok,
                                               const float *__restrict__ pos, int n_past, float *__restrict__ x) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (size_t)n_tok * w.nb) return;
  const int bl = (int)(t % w.nb), i = (int)(t / w.nb);
  const int j = tok[i];
  const int g = j / RG, r = j % RG;
  const size_t si = sc_index(w, g, bl, r);
  const float d = h2f_exact(w.d[si]);
  const float m = has_min(DT) ? h2f_exact(w.m[si]) : 0.0f;
  const size_t n = (size_t)w.nb * QK;
  float *o = x + (size_t)i * n + (size_t)bl * QK;
  const float *p = pos + (size_t)(n_past + i) * n + (size_t)bl * QK;
  for (int e = 0; e < QK; ++e) o[e] = __fadd_rn(__fadd_rn(__fmul_rn(d, (float)weight_q<DT>(w, g, bl, r, e)), m), p[e]);
}

// y = layernorm(x) row by row (src/tensor.rs:274-287): mean, mean of squared
// deviations, inv = 1 / sqrt(var + 1e-5), (x - mean) * inv * w + b; the sums
// in tree order.  One workgroup per row.  With r != NULL the residual add
// comes first: x += r (stored back), then y = layernorm(x).
__global__ __launch_bounds__(256) void k_layernorm(float *__restrict__ x, int n, const float *__restrict__ w,
                                                   const float *__restrict__ b, float *__restrict__ y,
                                                   const float *__restrict__ r) {
  __shared__ float part[2][4];
  const int row = blockIdx.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  float *xr = x + (size_t)row * n;
  if (r) {
    const float *rr = r + (size_t)row * n;
    for (int c = t; c < n; c += 256) xr[c] = xr[c] + rr[c];
    __syncthreads();
  }
  auto reduce = [&](float v, int slot) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
    if (lane == 0) part[slot][wv] = v;
    __syncthreads();
    return (part[slot][0] + part[slot][1]) + (part[slot][2] + part[slot][3]);
  };
  float s = 0.0f;
  for (int c = t; c < n; c += 256) s += xr[c];
  const float mean = __fdiv_rn(reduce(s, 0), (float)n);
  s = 0.0f;
  for (int c = t; c < n; c += 256) {
    const float d = xr[c] - mean;
    s += d * d;
  }
  const float var = __fdiv_rn(reduce(s, 1), (float)n);
  const float inv = __fdiv_rn(1.0f, __fsqrt_rn(var + 1e-5f));
  float *yr = y + (size_t)row * n;
  for (int c = t; c < n; c += 256) yr[c] = (xr[c] - mean) * inv * w[c] + b[c];
}

// h = gelu(h), the tanh form of src/tensor.rs:289-305 in its order
__global__ __launch_bounds__(256) void k_gelu(float *__restrict__ h, size_t n) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n) {
    const float v = h[t];
    const float inner = 0.7978846f * (v + 0.044715f * v * v * v);
    h[t] = 0.5f * v * (1.0f + tanhf(inner));
  }
}

#endif  // __HIPCC__

}  // namespace rw
