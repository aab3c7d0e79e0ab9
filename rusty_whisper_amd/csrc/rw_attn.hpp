// rw_attn.hpp -- multi-head attention on gfx950 (device code).
//
// out[t_q, n_state] = concat_h softmax(q_h k_h^T / sqrt(64) + mask) v_h, as
// mha_split_kv (src/encoder.rs:48-80) computes it in f32.  Two launches:
//
//   k_attn_split   q, k and v (f32) -> f16 pairs, one launch
//        x = hi + lo (hi = f16(x), lo = f16(x - hi)), head-major planes:
//        q, k  [head][t_pad][64]      (q pre-scaled by 1/8, exact)
//        v^T   [head][64][t_kv_pad]   kv positions permuted in 16-blocks
//   k_attn    one workgroup per (64 query rows, head), two wavefronts that
//        split the kv blocks between them and meet in LDS at the end.
//
// Precision.  Every product runs on v_mfma_f32_32x32x16_f16 as three f16
// products, hi*hi + hi*lo + lo*hi, accumulated in f32: each operand keeps
// 22 of f32's 24 significant bits and the dropped lo*lo term is below 2^-22
// of the product, so outputs stay within about 1e-6 (relative to the row) of
// the exact result, like the reference's f32 arithmetic.  Probabilities
// enter as 2^12 p so that small ones keep their f16 bits.  Inputs must stay
// below f16's 65504 in magnitude (whisper's projections are far below it);
// inputs below about 1e-3 lose a few bits to f16 subnormal residuals.  The
// softmax is online (running maximum and sum per query row, rescaled per
// block) in f32, which is the reference's max / exp / sum / divide reordered.
//
// Layouts inside k_attn.  The score block is computed transposed, S^T = K Q^T
// (32 kv x 32 queries): lane (h, n) then holds 16 kv entries of query n, so a
// query row's maximum and sum are in-lane plus one exchange with lane n+32.
// The output is accumulated transposed as well, O^T = V^T P^T, so the
// per-block rescale of a query column is one multiplier per lane.  P^T's
// registers feed that MFMA's B operand directly: lane half h holds kv
// 4h..4h+3 and 8+4h..8+4h+3 of each 16, and the v^T plane stores each
// 16-block of kv positions in that order (attn_vpos).
#pragma once
#include <stdint.h>

#include "rw_layout.hpp"

namespace rw {

constexpr int ATT_DH = 64;   // head size (every whisper model)
constexpr int ATT_KVB = 32;  // kv rows per block
constexpr int ATT_QT = 2;    // 32-query tiles per workgroup
constexpr int ATT_QB = 32 * ATT_QT;
#ifndef ATT_MAX_SPLIT_N
#define ATT_MAX_SPLIT_N 32
#endif
constexpr int ATT_MAX_SPLIT = ATT_MAX_SPLIT_N;  // kv runs of one (query block, head) at most
static_assert(ATT_MAX_SPLIT < 128, "k_attn packs the run count into 7 bits");

// kv index (within a 16-block) stored at position p of the v^T plane: the
// middle quads swap (an involution)
RW_HD inline int attn_vpos(int p) {
  const int qd = (p >> 2) & 3;
  return qd == 1 ? p + 4 : qd == 2 ? p - 4 : p;
}

struct AttnPlanes {
  const uint16_t *qh, *ql, *kh, *kl, *vh, *vl;
  int tq_pad, tkv_pad;
};

#if defined(__HIPCC__)

typedef _Float16 att_v8h __attribute__((ext_vector_type(8)));
typedef float att_v16f __attribute__((ext_vector_type(16)));

// x = hi + lo, both f16
constexpr float ATT_PS = 4096.0f;
__device__ inline void att_split(float x, uint16_t &hi, uint16_t &lo) {
  const _Float16 h = (_Float16)x;
  const _Float16 l = (_Float16)(x - (float)h);
  hi = __builtin_bit_cast(uint16_t, h);
  lo = __builtin_bit_cast(uint16_t, l);
}

// q or k rows -> [head][t_pad][64] f16 pairs; rows >= t are zeros.  Item
// idx covers 8 consecutive values of one row and head.
__device__ inline void att_split_rows(size_t idx, const float *__restrict__ x, int ld, int t, int t_pad,
                                      float scale, uint16_t *__restrict__ hi, uint16_t *__restrict__ lo) {
  const int c = (int)(idx & 7);
  const size_t hr = idx >> 3;  // head * t_pad + row
  const int row = (int)(hr % t_pad), head = (int)(hr / t_pad);
  float v[8];
  if (row < t) {
    const float4 *src = reinterpret_cast<const float4 *>(x + (size_t)row * ld + head * ATT_DH + c * 8);
    const float4 a = src[0], b = src[1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.0f;
  }
  uint16_t h8[8], l8[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) att_split(v[e] * scale, h8[e], l8[e]);
  const size_t o = hr * ATT_DH + c * 8;
  *reinterpret_cast<uint4 *>(hi + o) = *reinterpret_cast<const uint4 *>(h8);
  *reinterpret_cast<uint4 *>(lo + o) = *reinterpret_cast<const uint4 *>(l8);
}

// v^T [head][64][t_pad] f16 pairs: kv positions permuted by attn_vpos within
// each 16-block; kv >= t are zeros.
// v -> v^T pairs, one workgroup per (head, 64 kv positions): the 64 x 64
// values are read as row-contiguous 16-byte loads, split, and transposed
// through LDS (each position at its attn_vpos place, an involution), then
// written as 128-byte runs of positions per d and plane.  `sh` holds 2 x 64
// rows of ATT_VT_LD halves.
constexpr int ATT_VT_KV = 64, ATT_VT_LD = ATT_VT_KV + 8;
__device__ inline int att_vt_tiles(int t_pad) { return (t_pad + ATT_VT_KV - 1) / ATT_VT_KV; }
__device__ inline void att_split_vt_tile(int tile, const float *__restrict__ v, int ld, int t, int t_pad,
                                         uint16_t *__restrict__ hi, uint16_t *__restrict__ lo, uint16_t *sh) {
  const int nt = att_vt_tiles(t_pad);
  const int head = tile / nt, kv0 = (tile % nt) * ATT_VT_KV;
  const int th = threadIdx.x, d4 = th & 15;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int row = (th >> 4) + 16 * u, kv = kv0 + row;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (kv < t) x = *reinterpret_cast<const float4 *>(v + (size_t)kv * ld + head * ATT_DH + 4 * d4);
    const int pos = (row & ~15) | attn_vpos(row & 15);
    const float xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint16_t hb, lb;
      att_split(xs[e], hb, lb);
      sh[(4 * d4 + e) * ATT_VT_LD + pos] = hb;
      sh[(ATT_DH + 4 * d4 + e) * ATT_VT_LD + pos] = lb;
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int c = th + 256 * u;  // (plane, d, 8 positions)
    const int pl = c >> 9, d = (c >> 3) & 63, ch = c & 7;
    if (kv0 + 8 * ch < t_pad) {
      const uint4 w = *reinterpret_cast<const uint4 *>(sh + (pl * ATT_DH + d) * ATT_VT_LD + 8 * ch);
      *reinterpret_cast<uint4 *>((pl ? lo : hi) + ((size_t)head * ATT_DH + d) * t_pad + kv0 + 8 * ch) = w;
    }
  }
}

// All three splits in one launch: workgroups [0, wq) split q (scaled by
// 1/8, exact), [wq, wq + wk) split k, the rest split v into v^T
// (n_head * att_vt_tiles(tkv_pad) workgroups).
__global__ __launch_bounds__(256) void k_attn_split(const float *__restrict__ q, int ldq, int t_q,
                                                    const float *__restrict__ k, int ldk, const float *__restrict__ v,
                                                    int ldv, int t_kv, AttnPlanes P, int n_head, int wq, int wk) {
  const int bx = blockIdx.x;
  if (bx < wq) {
    const size_t idx = (size_t)bx * 256 + threadIdx.x;
    if (idx < (size_t)n_head * P.tq_pad * 8)
      att_split_rows(idx, q, ldq, t_q, P.tq_pad, 0.125f, const_cast<uint16_t *>(P.qh), const_cast<uint16_t *>(P.ql));
  } else if (bx < wq + wk) {
    const size_t idx = (size_t)(bx - wq) * 256 + threadIdx.x;
    if (idx < (size_t)n_head * P.tkv_pad * 8)
      att_split_rows(idx, k, ldk, t_kv, P.tkv_pad, 1.0f, const_cast<uint16_t *>(P.kh), const_cast<uint16_t *>(P.kl));
  } else {
    __shared__ __align__(16) uint16_t sh[2 * ATT_DH * ATT_VT_LD];
    const int tile = bx - wq - wk;
    if (tile < n_head * att_vt_tiles(P.tkv_pad))  // uniform: the whole workgroup
      att_split_vt_tile(tile, v, ldv, t_kv, P.tkv_pad, const_cast<uint16_t *>(P.vh), const_cast<uint16_t *>(P.vl),
                        sh);
  }
}

// Several decoding states' one-token steps in one self-attention: plane
// "head" b * n_head + h is head h of beam b, so one k_attn launch over
// n_beams * n_head heads serves every beam (each attends to its own cache).
constexpr int ATT_MAX_BEAMS = 8;
struct BeamCaches {
  float *k[ATT_MAX_BEAMS];  // beam b's f32 key cache [n_ctx][n]
  float *v[ATT_MAX_BEAMS];  // and value cache
};

// out rows [0, t) x columns [0, cols) = 0 (attention over no keys)
__global__ __launch_bounds__(256) void k_attn_zero(float *__restrict__ out, int ld, int t, int cols) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx < (size_t)t * cols) out[(idx / cols) * ld + idx % cols] = 0.0f;
}

__device__ inline att_v8h att_ld(const uint16_t *p) {
  return __builtin_bit_cast(att_v8h, *reinterpret_cast<const uint4 *>(p));
}

// c += ah bh + ah bl + al bh
__device__ inline void att_mma3(att_v8h ah, att_v8h al, att_v8h bh, att_v8h bl, att_v16f &c) {
  c = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bl, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bh, c, 0, 0, 0);
}

// One kv block's operands for one wavefront: K rows as the A operand of S^T
// (4 steps of 16 of the head's 64 values), v^T rows as the A operand of O^T
// (2 row tiles of 32 values x 2 steps of 16 kv).
struct AttK {
  att_v8h kh[4], kl[4];
};
struct AttV {
  att_v8h vh[2][2], vl[2][2];
};

__device__ inline void att_load_k(const AttnPlanes &P, int head, int blk, int h, int n, AttK &o) {
  const size_t krow = ((size_t)head * P.tkv_pad + (size_t)blk * ATT_KVB + n) * ATT_DH + 8 * h;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    o.kh[s] = att_ld(P.kh + krow + 16 * s);
    o.kl[s] = att_ld(P.kl + krow + 16 * s);
  }
}

__device__ inline void att_load_v(const AttnPlanes &P, int head, int blk, int h, int n, AttV &o) {
#pragma unroll
  for (int dt = 0; dt < 2; ++dt) {
    const size_t vrow = ((size_t)head * ATT_DH + dt * 32 + n) * P.tkv_pad + (size_t)blk * ATT_KVB + 8 * h;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      o.vh[dt][s] = att_ld(P.vh + vrow + 16 * s);
      o.vl[dt][s] = att_ld(P.vl + vrow + 16 * s);
    }
  }
}

// The same K and v^T operands straight from f32 rows (kf, vf with row
// strides ldk, ldv; rows >= t_kv are zeros), for calls that do not split K
// and V into planes first: the loads (raw) and the split (att_split, the
// values k_attn_split stores) are separate, so the loads can run ahead.
struct AttKRaw {
  float4 x[4][2];
};
struct AttVRaw {
  float x[2][2][8];
};
// (last: the newest kv row, t_kv - 1, comes from there instead of kf / vf)
__device__ inline void att_load_k_raw(const float *kf, int ldk, int t_kv, int head, int blk, int h, int n,
                                      AttKRaw &o, const float *last = nullptr) {
  // lane (h, n): kv row 32 blk + n, values 8h + 16s .. + 7
  const int row = min(blk * ATT_KVB + n, t_kv - 1);
  const float *src = (last && row == t_kv - 1 ? last : kf + (size_t)row * ldk) + head * ATT_DH + 8 * h;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    o.x[s][0] = *reinterpret_cast<const float4 *>(src + 16 * s);
    o.x[s][1] = *reinterpret_cast<const float4 *>(src + 16 * s + 4);
  }
}
__device__ inline void att_split_k(const AttKRaw &x, bool live, AttK &o) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const float v[8] = {x.x[s][0].x, x.x[s][0].y, x.x[s][0].z, x.x[s][0].w,
                        x.x[s][1].x, x.x[s][1].y, x.x[s][1].z, x.x[s][1].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint16_t hb, lb;
      att_split(live ? v[e] : 0.0f, hb, lb);
      o.kh[s][e] = __builtin_bit_cast(_Float16, hb);
      o.kl[s][e] = __builtin_bit_cast(_Float16, lb);
    }
  }
}
__device__ inline void att_load_v_raw(const float *vf, int ldv, int t_kv, int head, int blk, int h, int n,
                                      AttVRaw &o, const float *last = nullptr) {
  // lane (h, n): value d = 32 dt + n of the kv rows that the v^T plane keeps
  // at positions 32 blk + 16 s + 8 h + e (attn_vpos order within 16)
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int kv = blk * ATT_KVB + 16 * s + attn_vpos(8 * h + e), row = min(kv, t_kv - 1);
        const float x = (last && row == t_kv - 1 ? last : vf + (size_t)row * ldv)[head * ATT_DH + dt * 32 + n];
        o.x[dt][s][e] = kv < t_kv ? x : 0.0f;
      }
}
__device__ inline void att_split_v(const AttVRaw &x, AttV &o) {
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint16_t hb, lb;
        att_split(x.x[dt][s][e], hb, lb);
        o.vh[dt][s][e] = __builtin_bit_cast(_Float16, hb);
        o.vl[dt][s][e] = __builtin_bit_cast(_Float16, lb);
      }
}

// Workgroup (blockIdx.x, blockIdx.y) = (ATT_QB query rows from q0, head).
// Wavefront w takes kv blocks w, w + 2, ...; a causal query row i (at
// absolute position t_kv - t_q + i) sees kv rows up to its position.
//
// Split kv (few query blocks, e.g. one decoding step): with part != NULL,
// workgroup z of gridDim.z takes the z-th run of the kv blocks and writes
// its unnormalized O (2^12-scaled), running maximum and sum to part;
// k_attn_combine merges the runs.
//
// With qf != NULL the queries come as f32 rows (qf, ldq) and are scaled and
// split here, exactly as k_attn_split would store them (P.qh, P.ql unused):
// the decoder's cross-attention, whose K and v^T planes are kept, then needs
// no split launch.  QT: 32-query tiles per workgroup (2, or 1 for calls of at
// most 32 query rows: a decoding step then does half the products and
// softmax work; a query row's arithmetic does not depend on QT).
// ROWS: K and V come as f32 rows too (kf, vf) and are split
// here as well (the P planes are unused): calls of one query block (a
// decoding step's self-attention over its cache) then need no split launch;
// the operands are the planes' values, so the results are the same bits.
// The scalars and row pointers lead the arguments: the first 14 dwords
// arrive in SGPRs when the waves start (kernarg preloading), so a decoding
// step's attention requests its rows without first reading the argument
// block; the planes (P) follow.  The grid comes as arguments too (gridDim
// is read from the argument block): nx = gridDim.x, gw = causal | gridDim.z
// << 1 | gridDim.y << 8.
// (defined with the decode GEMV: a block of 8 lanes x 4 values as row i's
// activation record of block bl)
__device__ void attn_block_records(uint8_t *rec, int i, int bl, int lt, int mr, float4 x, int off, bool write);

// BEAMS (with ROWS): several beams' self-attention, one query row per
// (beam, head) plane, plane b * n_head + h; its q row is qf + b n + 64 h, its
// K and V rows beam b's caches C.k[b], C.v[b] except the newest (row
// t_kv - 1), which comes from the step's new rows kf, vf [beams][n] and is
// stored into the caches at that row (by the kv split's first run).
// rec (BEAMS, no kv split): also the output rows' activation records for
// the next product.  rec_hd = heads per beam | offset term << 8 | beams << 16.
template <bool ROWS, int QT, bool BEAMS = false>
__global__ __launch_bounds__(128) void k_attn(int t_q, int t_kv, int gw, int nx, const float *__restrict__ qf,
                                              int ldq, const float *__restrict__ kf, int ldk,
                                              const float *__restrict__ vf, int ldv, float *__restrict__ out,
                                              int ld_out, float *__restrict__ part, AttnPlanes P,
                                              uint8_t *__restrict__ rec, int rec_hd, BeamCaches C) {
  const int causal = gw & 1, gz = (gw >> 1) & 127, gy = gw >> 8;
  constexpr int QB = 32 * QT;  // query rows per workgroup
  constexpr float LOG2E = 1.4426950408889634f;
  constexpr float NEG_INF = -__builtin_huge_valf();
  __shared__ __align__(16) float xo[QB * (ATT_DH + 4)];  // partial O^T exchange, then the output tile
  __shared__ float xm[QT * 64], xl[QT * 64];
  const int l = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = l >> 5, n = l & 31;
  // XCD-aware order: workgroup id % 8 is its XCD; each XCD takes one
  // contiguous range of (head, query block) in head-major order, so a
  // head's query blocks share their K and v^T planes through one L2
  int head, q0;
  {
    const int nqb = nx, total = nqb * gy;
    const int id = blockIdx.y * nqb + blockIdx.x;
    const int per = total / 8, rem = total % 8, xcd = id % 8, slot = id / 8;
    const int lin = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
    head = lin / nqb;
    q0 = (lin % nqb) * QB;
  }
  const int off = t_kv - t_q;  // absolute position of query row 0
  const int kv_end = causal ? min(t_kv, off + q0 + QB) : t_kv;
  const int nblk_all = (kv_end + ATT_KVB - 1) / ATT_KVB;
  const int cs = (nblk_all + gz - 1) / gz;                     // blocks per split
  const int b_begin = min(nblk_all, (int)blockIdx.z * cs);
  const int nblk = min(nblk_all, b_begin + cs);               // this workgroup: blocks [b_begin, nblk)

  att_v8h qh[QT][4], ql[QT][4];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const size_t qrow = ((size_t)head * P.tq_pad + q0 + qt * 32 + n) * ATT_DH + 8 * h;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (qf) {
        const int row = q0 + qt * 32 + n;
        float v[8];
        if (row < t_q) {
          const float4 *src = reinterpret_cast<const float4 *>(qf + (size_t)row * ldq + head * ATT_DH + 8 * h + 16 * s);
          const float4 a = src[0], b = src[1];
          v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          uint16_t hb, lb;
          att_split(v[e] * 0.125f, hb, lb);
          qh[qt][s][e] = __builtin_bit_cast(_Float16, hb);
          ql[qt][s][e] = __builtin_bit_cast(_Float16, lb);
        }
      } else {
        qh[qt][s] = att_ld(P.qh + qrow + 16 * s);
        ql[qt][s] = att_ld(P.ql + qrow + 16 * s);
      }
    }
  }
  att_v16f o[QT][2];  // O^T
  float m[QT], lsum[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    o[qt][0] = (att_v16f){};
    o[qt][1] = (att_v16f){};
    m[qt] = NEG_INF;
    lsum[qt] = 0.0f;
  }

  // K one block ahead; V is loaded at the top of its block and first used
  // after the scores and the softmax
  AttK cur, nxt;
  AttV vb;
  AttKRaw kr_cur, kr_nxt;  // ROWS: f32 K rows, split when their block comes
  AttVRaw vr;
  // this plane's K and V rows (BEAMS: its beam's caches and new row)
  const float *kfp = kf, *vfp = vf, *klast = nullptr, *vlast = nullptr;
  int hkv = head;
  if constexpr (BEAMS) {
    const int hpb = rec_hd & 255, bb = head / hpb;
    hkv = head - bb * hpb;
    kfp = C.k[bb];
    vfp = C.v[bb];
    klast = kf + (size_t)bb * ldk;
    vlast = vf + (size_t)bb * ldv;
    if (blockIdx.z == 0) {  // the new row into the caches (read from kf / vf in this launch)
      const int t = threadIdx.x & 63;
      if (threadIdx.x < 64) C.k[bb][(size_t)(t_kv - 1) * ldk + hkv * ATT_DH + t] = klast[hkv * ATT_DH + t];
      else C.v[bb][(size_t)(t_kv - 1) * ldv + hkv * ATT_DH + t] = vlast[hkv * ATT_DH + t];
    }
  }
  if (b_begin + wv < nblk) {
    if constexpr (ROWS) att_load_k_raw(kfp, ldk, t_kv, hkv, b_begin + wv, h, n, kr_cur, klast);
    else att_load_k(P, head, b_begin + wv, h, n, cur);
  }
  for (int b = b_begin + wv; b < nblk; b += 2) {
    if constexpr (ROWS) {
      att_load_v_raw(vfp, ldv, t_kv, hkv, b, h, n, vr, vlast);
      if (b + 2 < nblk) att_load_k_raw(kfp, ldk, t_kv, hkv, b + 2, h, n, kr_nxt, klast);
      att_split_k(kr_cur, b * ATT_KVB + n < t_kv, cur);
    } else {
      att_load_v(P, head, b, h, n, vb);
      if (b + 2 < nblk) att_load_k(P, head, b + 2, h, n, nxt);
    }
    // both query tiles' scores first, so the softmax of one tile can run on
    // the VALU while the matrix cores work on the other
    att_v16f s[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      s[qt] = (att_v16f){};
#pragma unroll
      for (int k = 0; k < 4; ++k) att_mma3(cur.kh[k], cur.kl[k], qh[qt][k], ql[qt][k], s[qt]);
    }
    if constexpr (ROWS) att_split_v(vr, vb);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      // lane (h, n): s[qt][i] = score of query q0 + 32 qt + n against kv
      // row 32 b + 8 (i / 4) + 4 h + i % 4
      const int tq0 = q0 + qt * 32;
      const bool partial = (b + 1) * ATT_KVB > t_kv || (causal && (b + 1) * ATT_KVB - 1 > off + tq0);
      if (partial) {
        const int qpos = off + tq0 + n;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kv = b * ATT_KVB + 8 * (i >> 2) + 4 * h + (i & 3);
          if (kv >= t_kv || (causal && kv > qpos)) s[qt][i] = NEG_INF;
        }
      }
      float mx = s[qt][0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[qt][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mnew = fmaxf(m[qt], mx);
      const float mu = mnew == NEG_INF ? 0.0f : mnew;  // a column with nothing visible yet
      float ps = 0.0f;
      att_v8h ph[2], pl[2];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = __builtin_amdgcn_exp2f((s[qt][i] - mu) * LOG2E);
        ps += p;
        // P enters the products as 2^12 p, so that small probabilities keep
        // their f16 bits; the output is divided by 2^12 lsum at the end
        const float p12 = p * ATT_PS;
        const _Float16 ph1 = (_Float16)p12;
        ph[i >> 3][i & 7] = ph1;
        pl[i >> 3][i & 7] = (_Float16)(p12 - (float)ph1);
      }
      // rescale only when some column's maximum moved (rare after the
      // first blocks)
      if (__builtin_amdgcn_ballot_w64(mnew != m[qt])) {
        const float alpha = __builtin_amdgcn_exp2f((m[qt] - mu) * LOG2E);
        lsum[qt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) o[qt][dt] *= alpha;
      }
      m[qt] = mnew;
      lsum[qt] += ps;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int k = 0; k < 2; ++k) att_mma3(vb.vh[dt][k], vb.vl[dt][k], ph[k], pl[k], o[qt][dt]);
    }
    if constexpr (ROWS) kr_cur = kr_nxt;
    else cur = nxt;
  }

  // wavefront 1 hands its partial state to wavefront 0
  if (wv == 1) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) xo[((qt * 2 + dt) * 16 + i) * 64 + l] = o[qt][dt][i];
      xm[qt * 64 + l] = m[qt];
      xl[qt * 64 + l] = lsum[qt];
    }
  }
  __syncthreads();
  if (wv == 0) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const float m1 = xm[qt * 64 + l], l1 = xl[qt * 64 + l];
      const float mm = fmaxf(m[qt], m1);
      const float mu = mm == NEG_INF ? 0.0f : mm;
      const float s0 = __builtin_amdgcn_exp2f((m[qt] - mu) * LOG2E), s1 = __builtin_amdgcn_exp2f((m1 - mu) * LOG2E);
      float lt = lsum[qt] * s0 + l1 * s1;
      lt += __shfl_xor(lt, 32);
      const float inv = part ? 1.0f : 1.0f / (lt * ATT_PS);
      if (part && h == 0 && q0 + qt * 32 + n < t_q) {
        const size_t pr = ((size_t)blockIdx.z * gy + head) * P.tq_pad + q0 + qt * 32 + n;
        float *pml = part + (size_t)gz * gy * P.tq_pad * ATT_DH;
        pml[2 * pr] = mm;
        pml[2 * pr + 1] = lt;
      }
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          o[qt][dt][i] = (o[qt][dt][i] * s0 + xo[((qt * 2 + dt) * 16 + i) * 64 + l] * s1) * inv;
    }
  }
  __syncthreads();
  // the output tile [64 queries][64 d] through LDS, then row-contiguous stores
  constexpr int LD = ATT_DH + 4;
  if (wv == 0) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<float4 *>(&xo[(qt * 32 + n) * LD + dt * 32 + 8 * g + 4 * h]) =
              make_float4(o[qt][dt][4 * g], o[qt][dt][4 * g + 1], o[qt][dt][4 * g + 2], o[qt][dt][4 * g + 3]);
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < QB * 16 / 128; ++it) {
    const int c = it * 128 + (int)threadIdx.x;
    const int row = c >> 4, c4 = c & 15;
    if (q0 + row < t_q) {
      float *dst = part ? part + (((size_t)blockIdx.z * gy + head) * P.tq_pad + q0 + row) * ATT_DH + 4 * c4
                        : out + (size_t)(q0 + row) * ld_out + head * ATT_DH + 4 * c4;
      *reinterpret_cast<float4 *>(dst) = *reinterpret_cast<const float4 *>(&xo[row * LD + 4 * c4]);
    }
    // the one query row is threads 0-15 of the first pass: each 8 of them
    // one 32-column block (every lane of the wavefront quantizes its values)
    if (it == 0 && rec && threadIdx.x < 64) {
      const int hpb = rec_hd & 255;
      attn_block_records(rec, head / hpb, (head % hpb) * 2 + (c4 >> 3), c4 & 7, rec_hd >> 16,
                         *reinterpret_cast<const float4 *>(&xo[row * LD + 4 * c4]), (rec_hd >> 8) & 255,
                         q0 + row < t_q && row == 0);
    }
  }
}

// Merge nsplit runs of k_attn: out = sum_z O_z 2^(m_z - m) / (2^12 sum_z l_z
// 2^(m_z - m)), m the largest run maximum (runs that saw nothing have
// m = -inf and weigh 0).  One thread per (query, head, d).
// (defined with the decode GEMV: one query row's block of the output as the
// next product's activation record)
__device__ void combine_records(uint8_t *rec, int row, int col, int mr, float x, int off);

// With rec: also each query row's 32-column blocks of the output as
// activation records of the next product (its offset term `rec_off`), for
// 2-8 query rows; a wavefront holds one (row, head), two blocks.
__global__ __launch_bounds__(256) void k_attn_combine(const float *__restrict__ part, int nsplit, int n_head,
                                                      int tq_pad, int t_q, float *__restrict__ out, int ld_out,
                                                      uint8_t *__restrict__ rec, int rec_off) {
  constexpr float LOG2E = 1.4426950408889634f;
  constexpr float NEG_INF = -__builtin_huge_valf();
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)t_q * n_head * ATT_DH) return;
  const int d = (int)(idx % ATT_DH);
  const int head = (int)((idx / ATT_DH) % n_head), q = (int)(idx / ((size_t)ATT_DH * n_head));
  const float *pml = part + (size_t)nsplit * n_head * tq_pad * ATT_DH;
  // every run's maximum, sum and output value requested at once (one memory
  // round trip), then folded in run order
  float mz[ATT_MAX_SPLIT], lz[ATT_MAX_SPLIT], oz[ATT_MAX_SPLIT];
#pragma unroll
  for (int z = 0; z < ATT_MAX_SPLIT; ++z) {
    mz[z] = NEG_INF, lz[z] = 0.0f, oz[z] = 0.0f;
    if (z < nsplit) {
      const size_t pr = ((size_t)z * n_head + head) * tq_pad + q;
      mz[z] = pml[2 * pr];
      lz[z] = pml[2 * pr + 1];
      oz[z] = part[pr * ATT_DH + d];
    }
  }
  float mx = NEG_INF;
#pragma unroll
  for (int z = 0; z < ATT_MAX_SPLIT; ++z) mx = fmaxf(mx, mz[z]);
  const float mu = mx == NEG_INF ? 0.0f : mx;
  float num = 0.0f, den = 0.0f;
#pragma unroll
  for (int z = 0; z < ATT_MAX_SPLIT; ++z) {
    const float w = __builtin_amdgcn_exp2f((mz[z] - mu) * LOG2E);
    if (z < nsplit && w > 0.0f) {  // a run that saw no key holds no output
      num += oz[z] * w;
      den += lz[z] * w;
    }
  }
  const float y = num / (den * ATT_PS);
  out[(size_t)q * ld_out + head * ATT_DH + d] = y;
  if (rec) combine_records(rec, q, head * ATT_DH + d, t_q, y, rec_off);  // whole wavefronts (uniform)
}

#endif  // __HIPCC__

}  // namespace rw
