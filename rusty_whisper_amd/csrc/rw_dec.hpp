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

// x[i] = token_embedding.row_f32(tok[i]) + positional[n_past + i * pos_step]
// (src/decoder.rs:122-135): the quantized row dequantized as d * q + m (two
// roundings), then the position added.  pos_step is 1 for a prompt's
// consecutive tokens and 0 for one token of each of several beams.  One
// thread per (token, block).
template <int DT>
__global__ __launch_bounds__(256) void k_embed(WeightView w, const int *__restrict__ tok, int n_tok,
                                               const float *__restrict__ pos, int n_past, int pos_step,
                                               float *__restrict__ x) {
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
  const float *p = pos + (size_t)(n_past + i * pos_step) * n + (size_t)bl * QK;
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

// h = gelu(h) (src/tensor.rs:289-305; rw_kernels.hpp's gelu)
__global__ __launch_bounds__(256) void k_gelu(float *__restrict__ h, size_t n) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n) h[t] = gelu(h[t]);
}

constexpr int TOPK_MAX = 16;  // candidates per row of the top-k kernels

// Block-wide reductions of one value per thread (256 threads, 4 wavefronts)
__device__ inline float block_fmax(float v, float *scratch) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o));
  __syncthreads();  // scratch may hold the previous reduction's values
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(scratch[0], scratch[1]), fmaxf(scratch[2], scratch[3]));
}
__device__ inline float block_fsum(float v, float *scratch) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  return (scratch[0] + scratch[1]) + (scratch[2] + scratch[3]);
}
// (v, i) beats (bv, bi): larger v, or equal v and smaller i
__device__ inline bool topk_before(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

// log_softmax of each row (src/transcribe.rs:482-486: the maximum, lse =
// max + ln(sum exp(v - max)), lp = v - lse) and its top_k
// (src/transcribe.rs:672-685).  top_k scans the log-probs in id order,
// skips exactly -inf, and inserts (lp, id) ahead of every entry with an
// equal log-prob while the list has room or lp beats its last entry, then
// truncates to k.  With v* the k-th largest log-prob and g the number of
// larger ones, that keeps every entry above v*, and of the entries equal to
// v* those admitted (fewer than k entries >= v* precede them in id order)
// minus the oldest ones pushed out later: the last k - g admitted.  The
// list runs by log-prob, equal ones later id first.
// Three launches over chunks of TOPK_CHUNK logits (rows x chunks
// workgroups): k_topk_stats (each chunk's maximum and sum of exp(v - max)),
// k_topk_chunk (the row's lse from those partials, in one fixed order, then
// the chunk's first 2k - 1 entries in the order (lp desc, id asc)) and
// k_topk_merge (per row, v* and g from the chunks' picks, the admitted
// entries equal to v* in id order, and the list in the reference's order).
// A chunk holds at most g <= k - 1 entries above v*, so its first 2k - 1
// picks hold those and its first k entries equal to v*, which include every
// one of them the scan can admit: the merge is exact.
// A row holding NaN or +inf, or only -inf, has a NaN lse (as the reference
// computes it), so every log-prob is NaN; the scan then admits ids
// 0 .. k - 1, each ahead of the last, and keeps them with NaN log-probs.
// The sum runs in tree order, so lse (and every lp) can differ from the
// reference's sequential sum in its last bit.
constexpr int TOPK_CHUNK = 2048;  // logits per workgroup (8 per thread)
constexpr int TOPK_MAX_CHUNKS = 64;

__global__ __launch_bounds__(256) void k_topk_stats(const float *__restrict__ logits, int n, float *__restrict__ pm,
                                                    float *__restrict__ ps) {
  __shared__ float sf[4];
  const int c = blockIdx.x, row = blockIdx.y, nc = gridDim.x, t = threadIdx.x;
  const float *x = logits + (size_t)row * n;
  const int e0 = c * TOPK_CHUNK, e1 = min(n, e0 + TOPK_CHUNK);
  float v[TOPK_CHUNK / 256];
  float mx = -__builtin_huge_valf();
#pragma unroll
  for (int j = 0; j < TOPK_CHUNK / 256; ++j) {
    const int e = e0 + j * 256 + t;
    v[j] = e < e1 ? x[e] : -__builtin_huge_valf();
    mx = fmaxf(mx, v[j]);
  }
  mx = block_fmax(mx, sf);
  // an all -inf chunk (suppressed tokens) adds nothing; NaN, and +inf
  // (inf - inf), make the sum NaN as in the reference
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < TOPK_CHUNK / 256; ++j)
    if (e0 + j * 256 + t < e1 && v[j] != -__builtin_huge_valf()) sum += expf(v[j] - mx);
  sum = block_fsum(sum, sf);
  if (t == 0) {
    pm[(size_t)row * nc + c] = mx;
    ps[(size_t)row * nc + c] = sum;
  }
}

// the row's lse from its chunks' (maximum, sum) pairs: the maximum of the
// maxima, then sum_c s_c exp(m_c - M) in chunk order.  A chunk of NaNs only
// (maximum -inf, sum NaN) still makes it NaN, and so does a row of -inf
// only, whose reference maximum -inf gives -inf - -inf = NaN.
__device__ inline float topk_lse(const float *pm, const float *ps, int nc) {
  float M = -__builtin_huge_valf();
  for (int c = 0; c < nc; ++c) M = fmaxf(M, pm[c]);
  if (M == -__builtin_huge_valf()) return __builtin_nanf("");
  float S = 0.0f;
  for (int c = 0; c < nc; ++c)
    if (pm[c] > -__builtin_huge_valf() || ps[c] != ps[c]) S += ps[c] * expf(pm[c] - M);
  return M + logf(S);
}

// the block-wide first (v, i) in the selection order (lp desc, id asc)
__device__ inline void block_topk_argmax(float &bv, int &bi, float *rv, int *ri) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (topk_before(ov, oi, bv, bi)) bv = ov, bi = oi;
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) rv[threadIdx.x >> 6] = bv, ri[threadIdx.x >> 6] = bi;
  __syncthreads();
  bv = rv[0], bi = ri[0];
#pragma unroll
  for (int w = 1; w < 4; ++w)
    if (topk_before(rv[w], ri[w], bv, bi)) bv = rv[w], bi = ri[w];
}

// k rounds over the values a thread holds (`cnt` of them): each round picks
// the block's first entry after the previous pick; picks go to (ov, oi)[0, k),
// padded with (-inf, INT32_MAX).  Returns the number picked.
template <int PER>
__device__ inline int topk_rounds(const float (&lp)[PER], const int (&id)[PER], int k, float *ov, int *oi,
                                  float *rv, int *ri) {
  constexpr float NEG_INF = -__builtin_huge_valf();
  float pv = __builtin_huge_valf();
  int pi = -1, got = 0;
  for (int r = 0; r < k; ++r) {
    float bv = NEG_INF;
    int bi = INT32_MAX;
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (lp[j] > NEG_INF && topk_before(pv, pi, lp[j], id[j]) && topk_before(lp[j], id[j], bv, bi))
        bv = lp[j], bi = id[j];
    block_topk_argmax(bv, bi, rv, ri);
    if (bi == INT32_MAX) break;  // no candidate left (uniform)
    if (threadIdx.x == 0) ov[r] = bv, oi[r] = bi;
    pv = bv, pi = bi;
    got = r + 1;
  }
  if (threadIdx.x == 0)
    for (int r = got; r < k; ++r) ov[r] = NEG_INF, oi[r] = INT32_MAX;
  return got;
}

__global__ __launch_bounds__(256) void k_topk_chunk(const float *__restrict__ logits, int n, int k,
                                                    const float *__restrict__ pm, const float *__restrict__ ps,
                                                    float *__restrict__ cv, int *__restrict__ ci) {
  __shared__ float rv[4];
  __shared__ int ri[4];
  const int c = blockIdx.x, row = blockIdx.y, nc = gridDim.x, t = threadIdx.x;
  const float lse = topk_lse(pm + (size_t)row * nc, ps + (size_t)row * nc, nc);
  const float *x = logits + (size_t)row * n;
  const int e0 = c * TOPK_CHUNK, e1 = min(n, e0 + TOPK_CHUNK);
  constexpr int PER = TOPK_CHUNK / 256;
  float lp[PER];
  int id[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = e0 + j * 256 + t;
    id[j] = e;
    lp[j] = e < e1 ? x[e] - lse : -__builtin_huge_valf();  // NaN stays NaN and is never picked
  }
  const int cand = 2 * k - 1;
  const size_t o = ((size_t)row * nc + c) * cand;
  topk_rounds<PER>(lp, id, cand, cv + o, ci + o, rv, ri);
}

// the block-wide smallest of one int per thread
__device__ inline int block_imin(int v, int *scratch) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = min(v, __shfl_xor(v, o));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  return min(min(scratch[0], scratch[1]), min(scratch[2], scratch[3]));
}

__global__ __launch_bounds__(256) void k_topk_merge(int nc, int k, int n, const float *__restrict__ pm,
                                                    const float *__restrict__ ps, const float *__restrict__ cv,
                                                    const int *__restrict__ ci, uint32_t *__restrict__ ids,
                                                    float *__restrict__ lps) {
  constexpr float NEG_INF = -__builtin_huge_valf();
  __shared__ float rv[4];
  __shared__ int ri[4];
  __shared__ float pick_v[TOPK_MAX];
  __shared__ int pick_i[TOPK_MAX];
  __shared__ int adm[TOPK_MAX];
  const int row = blockIdx.x, t = threadIdx.x;
  uint32_t *oid = ids + (size_t)row * k;
  float *olp = lps + (size_t)row * k;
  const float lse = topk_lse(pm + (size_t)row * nc, ps + (size_t)row * nc, nc);
  if (lse != lse) {  // every log-prob NaN: ids min(k, n) - 1 .. 0
    const int kk = min(k, n);
    if (t < k) {
      oid[t] = t < kk ? (uint32_t)(kk - 1 - t) : 0xFFFFFFFFu;
      olp[t] = t < kk ? __builtin_nanf("") : NEG_INF;
    }
    return;
  }
  constexpr int PER = (TOPK_MAX_CHUNKS * (2 * TOPK_MAX - 1) + 255) / 256;
  float lp[PER];
  int id[PER];
  const int total = nc * (2 * k - 1);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = j * 256 + t;
    lp[j] = e < total ? cv[(size_t)row * total + e] : NEG_INF;
    id[j] = e < total ? ci[(size_t)row * total + e] : INT32_MAX;
  }
  // the k first in the order (lp desc, id asc): their values are the k
  // largest log-probs, so the last is v*
  const int got = topk_rounds<PER>(lp, id, k, pick_v, pick_i, rv, ri);
  __syncthreads();
  int g = got, a = 0;
  if (got == k) {
    const float vs = pick_v[k - 1];
    g = 0;
    while (g < k && pick_v[g] > vs) ++g;
    // the entries equal to v* in id order, while fewer than k entries >= v*
    // precede them (i earlier ones equal to v*, plus the larger ones before)
    int prev = -1;
    for (int i = 0; i < k; ++i) {
      int best = INT32_MAX;
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (lp[j] == vs && id[j] > prev && id[j] < best) best = id[j];
      best = block_imin(best, ri);
      if (best == INT32_MAX) break;  // uniform
      int before = i;
      for (int r = 0; r < g; ++r) before += pick_i[r] < best;
      if (before >= k) break;
      if (t == 0) adm[a] = best;
      ++a;
      prev = best;
    }
    __syncthreads();
  }
  if (t == 0) {
    // the entries above v* (all of them), equal log-probs later id first
    for (int x = 1; x < g; ++x)
      for (int y = x; y > 0 && pick_v[y] == pick_v[y - 1] && pick_i[y] > pick_i[y - 1]; --y) {
        const int ti = pick_i[y];
        pick_i[y] = pick_i[y - 1], pick_i[y - 1] = ti;
      }
    for (int r = 0; r < g; ++r) oid[r] = (uint32_t)pick_i[r], olp[r] = pick_v[r];
    if (got == k) {
      // then the last k - g admitted entries equal to v*, later id first
      for (int r = g; r < k; ++r) oid[r] = (uint32_t)adm[a - 1 - (r - g)], olp[r] = pick_v[k - 1];
    } else {
      for (int r = got; r < k; ++r) oid[r] = 0xFFFFFFFFu, olp[r] = NEG_INF;
    }
  }
}

#endif  // __HIPCC__

}  // namespace rw
